// C ABI of libvvllm_hip.so (include/vvllm_hip.h): device init, memory,
// caching allocator, weight mirror, dispatch of the linear path, grouped
// plans.  Every entry validates its arguments on the host, returns a
// vvh_status and records a message for vvh_last_error(); nothing exits the
// process (the reference exits on any CUDA error,
// src/backend/cuda_kernels.cu:11-21).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "pool.h"

using namespace vvh;

namespace vvh {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int fail_hip(hipError_t e, const char* what)
{
    if (e == hipErrorOutOfMemory)
        return fail(VVH_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
    return fail(VVH_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

}  // namespace vvh

namespace {

std::atomic<bool> g_init{false};
int g_device = -1;
int g_cu_count = 0;
std::atomic<int> g_override{K_AUTO};

#define REQUIRE_INIT()                                                              \
    do {                                                                            \
        if (!g_init.load()) return fail(VVH_ERR_NOT_INITIALIZED, "vvh_init has not succeeded"); \
    } while (0)

// ---- caching allocator over hipMalloc -------------------------------------
struct HipRaw final : RawAllocator {
    int alloc(void** p, std::size_t bytes) override
    {
        hipError_t e = hipMalloc(p, bytes);
        if (e == hipSuccess) return 0;
        (void)hipGetLastError();  // clear the sticky error of the failed allocation
        return e == hipErrorOutOfMemory ? 1 : 2;
    }
    int free(void* p) override { return hipFree(p) == hipSuccess ? 0 : 2; }
};
HipRaw g_raw;
CachingPool g_pool(&g_raw);

// ---- weight mirror --------------------------------------------------------
struct WeightEntry {
    const void* host_w = nullptr;      // key (null for device registrations)
    const void* host_scales = nullptr;
    const void* host_bias = nullptr;
    std::size_t N = 0, K = 0;
    void* base = nullptr;              // owned allocation (null if not owned)
    std::size_t bytes = 0;
    const int8_t* w = nullptr;
    const float* scales = nullptr;
    const float* bias = nullptr;
    int src_dtype = -1;                // vvh_weight_ingest: dtype of the host rows
};
std::mutex g_wmu;
std::unordered_map<vvh_weight, WeightEntry> g_weights;
std::unordered_map<const void*, vvh_weight> g_weight_by_host;
vvh_weight g_next_weight = 1;

// ---- plans ------------------------------------------------------------------
struct Plan {
    std::vector<LinArgs> args;   // host copy, launch order
    LinArgs* dev_table = nullptr;
    int act = 0, out = 0;
    bool grouped = false;        // one k_skinny_grouped launch
    int64_t total_blocks = 0;
    bool stream = false;         // one k_stream launch (kStreamList)
    bool dot = false;            // one k_dot_grouped launch
    int32_t* dev_block_prob = nullptr;
    bool x_in_lds = false;       // every problem's activations fit the block's LDS
    size_t lds_bytes = 0;
    StreamArgs sargs{};
    int depth = 0;
    int dot_depth = 4;           // k_dot_grouped ring depth: the largest dot_depth of the problems
    int max_m = 0;
    void* dev_stream = nullptr;  // tile_prob, list, list_off
    float* rope_freq = nullptr;  // RoPE epilogue: the pair frequencies of the q and k rows
    float* rope_cs = nullptr;    // RoPE epilogue: cosine and sine of positions [0, rope_cs_n)
    int64_t rope_cs_n = 0;
    // tables replaced by a later vvh_plan_set_rope or vvh_plan_set_rope_table:
    // a graph captured before may still read them, so they are freed with the plan
    std::vector<float*> rope_retired;
};
std::mutex g_pmu;
std::unordered_map<vvh_plan, Plan> g_plans;
vvh_plan g_next_plan = 1;

// ---- split-K workspace ------------------------------------------------------
// fp32 partial sums of split GEMMs and the partials of multi-block decode
// attention and sampling, one buffer per stream (calls on one stream run in
// order, so they can share it; calls on different streams never do).  Grown
// on demand to at least twice its size; a buffer it outgrows is retired, not
// freed, because a HIP graph captured earlier on the stream still holds its
// address in its kernel nodes (a replay must not touch freed memory).
// Retired buffers are freed by vvh_workspace_release or at process end.
struct Workspace {
    void* p = nullptr;
    std::size_t bytes = 0;
    std::vector<void*> retired;
    unsigned* cnt = nullptr;  // kAttnCounters arrival counters of the decode attention, zero between calls
};
std::mutex g_wsmu;
std::unordered_map<void*, Workspace> g_ws;

int workspace_for(void* stream, std::size_t bytes, float** out)
{
    std::lock_guard<std::mutex> lock(g_wsmu);
    Workspace& w = g_ws[stream];
    if (w.bytes < bytes) {
        const std::size_t nb = std::max({bytes, 2 * w.bytes, std::size_t(1) << 20});
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, nb);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail_hip(e, "workspace hipMalloc");
        }
        if (w.p) w.retired.push_back(w.p);
        w.p = p;
        w.bytes = nb;
    }
    *out = static_cast<float*>(w.p);
    return VVH_OK;
}

// The stream's decode-attention counters: allocated on first use and zeroed
// before this returns, by a kernel on a private non-blocking stream that the
// host waits for.  So they are zero for the first direct call and for the
// first replay alike, also when the first use happens inside a capture of
// `stream` (the private stream is not captured; no memset node is recorded);
// every call leaves them at zero again.
hipStream_t g_zero_stream[64] = {};

int counters_for(void* stream, unsigned** out)
{
    std::lock_guard<std::mutex> lock(g_wsmu);
    Workspace& w = g_ws[stream];
    if (!w.cnt) {
        if (g_device < 0 || g_device >= 64) return fail(VVH_ERR_UNSUPPORTED, "device %d out of range", g_device);
        hipStream_t& zs = g_zero_stream[g_device];
        if (!zs) {
            const hipError_t e = hipStreamCreateWithFlags(&zs, hipStreamNonBlocking);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                zs = nullptr;
                return fail_hip(e, "attention counters: private stream");
            }
        }
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, (std::size_t)kAttnCounters * sizeof(unsigned));
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail_hip(e, "attention counters hipMalloc");
        }
        int st = launch_zero_u32(static_cast<unsigned*>(p), kAttnCounters, zs);
        if (st == 0) st = (int)hipStreamSynchronize(zs);
        if (st != 0) {
            (void)hipGetLastError();
            (void)hipFree(p);
            return fail_hip((hipError_t)st, "attention counters zero launch");
        }
        w.cnt = static_cast<unsigned*>(p);
    }
    *out = w.cnt;
    return VVH_OK;
}

// ---- fixed scratch of vvh_linear_q8_dev_noalloc ------------------------------
// The split-K partial planes of the allocation-free entry point live in this
// file-scope device array: the code object holds it on every device the
// library runs on, until the process ends.  In host code its name is a
// host-side stand-in, not a device address; vvh_init looks up the device
// address once per device (hipGetSymbolAddress, with that device current)
// and every host use goes through g_scratch_ptr.  Every call on one device
// shares the array; the split GEMM writes every element of each partial
// plane before the reduction reads it, so nothing needs clearing between
// calls.
static __device__ __align__(256) unsigned char g_noalloc_scratch[VVH_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

int scratch_setup(int device)
{
    if (device < 0 || device >= kMaxDevices) return VVH_OK;  // vvh_linear_q8_dev_noalloc refuses such devices
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return VVH_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_noalloc_scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return fail_hip(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(noalloc scratch)");
    }
    g_scratch_ptr[device] = p;
    return VVH_OK;
}

// A call's workspace: the stream workspace (grown with hipMalloc) when src is
// null, else src's fixed buffer, which must be large enough.
int workspace_get(const WsSource* src, void* stream, std::size_t bytes, float** out)
{
    if (!src) return workspace_for(stream, bytes, out);
    if (bytes > src->bytes)
        return fail(VVH_ERR_UNSUPPORTED, "the call needs %zu bytes of workspace, more than the %zu of the "
                    "fixed buffer", bytes, src->bytes);
    *out = static_cast<float*>(src->fixed);
    return VVH_OK;
}

// Number of k splits for an M x N GEMM of `stages` 64-wide k stages.  A
// split GEMM pays a second launch and, per split, one M x N fp32 partial
// plane written by the GEMM and read back by the reduction, so it only pays
// for long reductions over few tiles: split when the 64 x 128 tiles would
// leave half of the CUs idle and K has at least 8 stages.  The
// count minimises a cost model fitted to sweeps of forced counts (graph
// replay): 0.25 us per k stage of a split block, 2.5 us for the
// reduction's launch, each plane at 1.6 TB/s, and 0.3 us per stage for an
// unsplit call.  Measured on 64 x 128 against 128 x 128 split tiles:
// 0.5B down (896 x 4864) at M = 128: 8 splits 11.77 us (128 x 128, 11
// splits: 14.64), M = 512: 4 splits 16.81 (6 on 128 x 128: 19.51), M = 64:
// 13 splits 11.13 (12.43); 1.5B down (1536 x 8960) at M = 16: 20 splits
// 11.83 (12.98), M = 64: 10 splits 14.25 (15.78), M = 256: 5 splits 19.74
// (22.0); 1.5B q/o at M = 64: 6 splits 9.73 (10.9), k/v: 12 splits 8.41
// (9.18).  Splits may be as short as 2 stages (k/v at M = 64: 12 splits
// against 6 at a floor of 4 stages, 9.18 against 10.12 us on 128 x 128).
// Split tiles of 64 x 64 (layout 5) enter the same model with a stage cost of
// 0.75 that of 64 x 128 (12 KB of LDS filled per stage instead of 16):
// measured with the counts it picks, down at M = 128 12.71 -> 11.70 us (7
// splits), 1.5B down at M = 64 14.40 -> 13.28 (10 splits), 1.5B q/o at M = 64
// / 128 9.85 / 10.36 -> 9.24 / 9.62, k/v at M = 64 / 256 8.56 / 9.20 -> 8.07 /
// 8.64; where 64 x 64 would halve the count (down at M = 512: 4 -> 2 splits,
// 16.83 -> 17.72 us; 1.5B down at M = 256: 19.79 -> 24.91) the model keeps
// 64 x 128.  *split_layout: the tile layout of a split call (4 or 5).
int gemm_splits(int64_t M, int64_t N, int64_t stages, int* split_layout)
{
    const int64_t cus = g_cu_count > 0 ? g_cu_count : 256;
    const int64_t tiles = ((M + 63) / 64) * ((N + 127) / 128);  // 64 x 128 tiles
    const double plane_bytes = (double)M * (double)N * 4.0;
    int64_t s = 1;
    int lay = 4;
    if (tiles * 2 <= cus && stages >= 8) {
        // unsplit: 64 x 64 tiles where they fit one round (gemm3_layout), about
        // 0.85 of the 64 x 128 time
        const bool one64 = ((M + 63) / 64) * ((N + 63) / 64) <= cus;
        double best = 0.3 * (double)stages * (one64 ? 0.85 : 1.0);
        for (const int L : {4, 5}) {
            const int64_t tl = L == 4 ? tiles : ((M + 63) / 64) * ((N + 63) / 64);
            const double f = L == 4 ? 1.0 : 0.75;
            const int64_t smax = std::min<int64_t>(cus / tl, stages / 2);
            for (int64_t c = 2; c <= smax; c++) {
                const int64_t kst = (stages + c - 1) / c, ce = (stages + kst - 1) / kst;  // no empty split
                if (ce == 1) continue;
                const int64_t rounds = (tl * ce + cus - 1) / cus;
                const double t = f * 0.25 * (double)(rounds * kst) + 2.5 + (double)ce * plane_bytes / 1.6e6;
                if (t < best) {
                    best = t;
                    s = c;
                    lay = L;
                }
            }
        }
    }
    s = std::max<int64_t>(1, std::min<int64_t>(s, stages));
    if (split_layout) *split_layout = lay;
    return (int)s;
}

// k_gemm3 tile numbering.  Each XCD (with its own L2) runs a contiguous
// range of about tiles * splits / 8 tiles.  Numbered row blocks fastest, the
// range covers many row blocks of few column blocks (the activation rows of
// all of them, the codes of few); column blocks fastest, the reverse.  The
// order whose range touches fewer operand bytes is taken: the down
// projection at M = 2048 (K = 4864: 32 x 7 tiles of 64 x 128) touches
// 18.0 MB per XCD row-fastest (28 row blocks of 622 KB of activations)
// against 6.8 MB column-fastest, and moved 155.7 MB of HBM traffic per call
// for 31.6 MB of algorithmic bytes row-fastest (rocprofv3 FETCH_SIZE).
// Measured (graph replay, every order forced in turn): that down projection
// 31.3 us row-fastest, 28.0 column-fastest; gate/up at M = 2048 (128 x 192,
// row-fastest kept) 30.5 against 31.5 us; the other configs[3] / configs[4]
// GEMM shapes alike within 0.3 us either way.
int gemm3_norder(int64_t M, int64_t N, int64_t act_row_halfs, int64_t krange_codes, int layout, int64_t splits)
{
    const int64_t bm = gemm3_tile_m(layout), bn = gemm3_tile_n(layout);
    const int64_t nbm = (M + bm - 1) / bm, nbn = (N + bn - 1) / bn;
    const int64_t tiles = nbm * nbn;
    const int64_t t = std::min(tiles, (tiles * splits + 7) / 8);  // one XCD's share, within one split
    const double a_blk = (double)bm * (double)act_row_halfs * 2.0, b_blk = (double)bn * (double)krange_codes;
    const double fp_m = (double)std::min(t, nbm) * a_blk + (double)((t + nbm - 1) / nbm) * b_blk;
    const double fp_n = (double)((t + nbn - 1) / nbn) * a_blk + (double)std::min(t, nbn) * b_blk;
    return fp_n < fp_m ? 1 : 0;
}

// k_gemm3 tile shape: split-K problems (few tiles, long K) take the layout
// gemm_splits chose (64 x 128 or 64 x 64).  Unsplit ones take 64 x 64 when
// those tiles give every block a CU of its own (gate/up N=4864 K=896 at
// M=128 8.42 -> 7.47 us against 64 x 128; q/k/v N=1152 at M=512 8.19 ->
// 7.19; 1.5B gate at M=64 12.04 -> 10.47; 1.5B q/o at M=256 11.48 -> 9.74;
// with two rounds of them, gate/up N=9728 at M=128, 8.64 -> 10.28, so not
// then), else 64 x 128 when those tiles give every block a CU of its
// own (then more CUs work than with 128-row tiles, each on half a tile:
// gate/up N=4864 K=896 at M=128 and 256, 10.5 -> 8.2 us; q/k/v N=1152 at
// M=512, 10.3 -> 8.0 us; with more 64-row tiles than CUs, two share a CU
// and the time rises: M=512 gate/up 10.7 -> 11.8 us); else 128 x 192 when
// it takes fewer rounds of blocks over the CUs than 128 x 128 by a margin
// that pays for its longer tiles (a 128 x 192 tile takes 1.33x as long as a
// 128 x 128 one on MI355X), else 128 x 128.  (128 x 128 as 8 waves of
// 64 x 32 measured the same as 4 waves of 128 x 32 at M=512: the loads
// into LDS, not latency within a SIMD, bound a block.)
int gemm3_layout(int64_t M, int64_t N, int splits, int split_layout)
{
    if (splits > 1) return split_layout;
    const int64_t cus = g_cu_count > 0 ? g_cu_count : 256;
    if (((M + 63) / 64) * ((N + 63) / 64) <= cus) return 5;
    if (((M + 63) / 64) * ((N + 127) / 128) <= cus) return 4;
    const int64_t nbm = (M + kGemmBM - 1) / kGemmBM;
    const int64_t r128 = (nbm * ((N + 127) / 128) + cus - 1) / cus;
    const int64_t r192 = (nbm * ((N + 191) / 192) + cus - 1) / cus;
    return 4 * r192 < 3 * r128 ? 1 : 3;
}

constexpr std::size_t kAlign = 256;
inline std::size_t align_up(std::size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
inline bool valid_dtype(int d) { return d == VVH_F32 || d == VVH_F16; }
inline std::size_t dsize(int d) { return d == VVH_F32 ? 4 : 2; }

// a*b without overflow past 2^62
bool mul_ok(uint64_t a, uint64_t b, uint64_t* r)
{
    if (a != 0 && b > (uint64_t(1) << 62) / a) return false;
    *r = a * b;
    return true;
}

// ---- persistent streaming decode (k_stream) --------------------------------
// Resident waves per CU of a streaming launch, and the smallest tile count
// worth a persistent launch (4 tiles per CU).
constexpr int kStreamWavesPerCu = 8;

int64_t stream_max_waves() { return (int64_t)(g_cu_count > 0 ? g_cu_count : 256) * kStreamWavesPerCu; }

// Pipeline depth the streaming kernel can use for problems whose smallest k
// step count is min_steps (0 = not eligible): 12 loads in flight per lane
// when every problem has 12 k steps, else 8.
int stream_depth(int64_t min_steps)
{
    if (min_steps < 8) return 0;
    return min_steps >= 12 ? 12 : 8;
}

// k_dot launches of at most ten blocks per CU take the variant that
// requests its weights and epilogue operands first: they are bounded by the
// latency of those loads, not by occupancy.  Without an input stage they also
// load the activations with the weights instead of staging them in LDS
// behind a barrier (same products in the same order, so the same results).
// Graph-replayed, Qwen2.5-0.5B shapes at M = 1: k/v 3.46 -> 2.88 us, q 3.76
// -> 3.23 us, o 4.04 -> 3.49 us, down 6.04 -> 4.96 us; gate/up (608 blocks)
// 5.74 -> 4.58 us, 18992 x 896 (594 blocks) 7.11 -> 6.28 us, the LM head
// (2374 blocks) 25.1 -> 24.7 us.  (With the old 8-deep ring, the early
// variant lost at 304 blocks, 5.36 -> 5.75 us: the ring held 64 VGPRs through
// the staging; with the ring sized to the k range it holds 16 or 32.)  At 20
// blocks per CU, which takes in the headline decode set (4752 blocks), that
// set measured the same as with staging.
constexpr int64_t kDotEarlyBlocksPerCu = 10;
bool dot_early(int64_t blocks) { return blocks <= (int64_t)(g_cu_count > 0 ? g_cu_count : 256) * kDotEarlyBlocksPerCu; }

// k_dot weight-ring depth: the wave's whole k range when it has 2 k steps
// (depth 2) or 5 to 7 (depth 7), else 4.  Each ring slot past the range
// re-reads a step (so that every wait in the pipeline has a fixed count),
// which costs issue time, and a ring deeper than the range refills.
// Graph-replayed at M = 1, against the earlier fixed 8: 2 steps per wave
// (Qwen2.5-0.5B q/k/v/o/gate/up at ksplit 4), depth 2: o 4.34 -> 3.93 us,
// gate/up 7.10 -> 5.70 us; 10 steps (0.5B down), depth 4: 6.57 -> 6.08 us;
// the headline decode set (one grouped launch), 56.2 -> 54.7 us per step over
// 20 steps.  7 steps (LM head, 151936 x 896): depth 8 25.5 us, 4 24.3 us, 7
// 23.6 us; depth 7 on longer ranges (down 896 x 4864, 1536 x 8960) lost 10%
// against 4.
int dot_depth(int64_t K, int ksplit)
{
    const int64_t steps = (K + kDotStep - 1) / kDotStep;
    const int64_t per_wave = (steps + ksplit - 1) / ksplit;
    return per_wave <= 2 ? 2 : (per_wave >= 5 && per_wave <= 7) ? 7 : 4;
}

// fp32 activations take the GEMM (on their split fp16 form) from this many
// rows on, when K % 64 == 0; below it k_gemv_f32, which streams the weights
// once per 8 rows (gate/up 4864 x 896, graph replay: M = 8 13.7 against
// 14.1 us on the GEMM, M = 16 17.0 against 14.2, M = 32 23.9 against 15.1).
constexpr std::size_t kGemmF32MinM = 16;

// Small-M fp16 dispatch, from a sweep of every family forced on each shape
// (us per call on the GPU, calls replayed from HIP graphs; the bench.py
// extras "decode_families" repeat part of it):
//                         M:  1     2     3     4     8     16
//   q 896 x 896      dot    3.22  3.73  4.59  4.66
//                    skinny 4.37  4.62  4.95  5.16  5.46
//                    gemm   8.59  8.57  8.74  8.83  8.91
//   down 896 x 4864  dot    5.05  6.77  8.25  8.89
//                    skinny 9.20  9.97 10.19 11.56 10.60 14.29
//                    gemm  10.36 10.42 10.57 10.84 10.81 10.99
//   gate_up 9728 x 896     dot 4.56 5.83 7.28 7.42, skinny 6.01 6.16 6.53 6.77 7.34
//   1.5B q/o 1536 x 1536   dot 3.67 4.41 5.39 5.55, skinny 5.26 5.40 5.99 6.25 5.58 5.56 (gemm 9.9 at 16)
//   1.5B gate_up 17920 x 1536  dot 9.39 10.86 14.85 15.31, skinny 10.88 11.59 11.93 12.23 15.14 18.33,
//                          gemm 13.78 14.30 14.20 13.87 14.40 14.43
//   1.5B down 1536 x 8960  dot 7.48 10.40 12.26 12.41, skinny 16.27 .. 22.82, gemm 12.8 .. 13.2
//   151936 x 896           dot 28.3 (M = 2) 34.1 (3), skinny 33.2 35.1 38.6 (8) 63.1 (16), gemm 54-56
// With k_dot's MFMA path for 3-4 rows (same graph replay), M = 3 / 4:
//   gate 4864 x 896 (304 tiles)          dot 4.22 4.36, skinny 5.59 5.87
//   gate_up 9728 x 896 (608 tiles)       dot 5.48 5.67, skinny 6.35 6.65
//   1.5B q/k/v 2048 x 1536 (128 tiles)   dot 4.18 4.34, skinny 5.82 6.06
//   1.5B gate_up 17920 x 1536 (1120)     dot 12.35 12.87, skinny 11.90 12.23
//   151936 x 896 (9496 tiles)            dot 38.6 40.2, skinny 34.9 35.8
// and with that path for 5-8 rows (8-row operands), M = 5 / 6 / 8:
//   o 896 x 896            dot 4.04 4.20 4.49, skinny 5.12 5.11 5.26, gemm 9.4-9.6
//   gate 4864 x 896        dot 5.15 5.34 5.63, skinny 6.02 6.13 6.28, gemm 10.0
//   gate_up 9728 x 896     dot 6.12 6.36 6.76, skinny 7.01 6.80 7.28, gemm 10.6
//   down 896 x 4864        dot 6.91 7.14 7.54, skinny 10.3-10.4, gemm 11.2
//   1.5B q/o 1536 x 1536   dot 4.80 5.02 5.32, skinny 5.96 5.28 5.31, gemm 9.7
//   1.5B down 1536 x 8960  dot 9.56 9.80 10.56, skinny 16.6-16.9, gemm 13.0-13.1
// and at M = 8 / 9 / 12 / 16 (k_dot's 16-row operands from M = 9):
//   o 896 x 896                  dot 4.53 5.83 6.29 6.94, skinny 5.25 5.33 4.57 4.67, gemm 9.6-9.8
//   gate 4864 x 896 (304 tiles)  dot 5.69 6.98 7.55 8.37, skinny 6.22 6.34 5.91 6.23, gemm 10.1-10.2
//   gate_up 9728 x 896 (608)     dot 6.84 8.05 8.70 9.66, skinny 7.31 7.37 7.26 7.61, gemm 10.65 10.7 10.78 8.10
//   down 896 x 4864 (56)         dot 7.61 8.56 9.46 10.77, skinny 10.4-11.1, gemm 11.25 11.37 11.4 11.43
//   1.5B q/o 1536 x 1536         dot 5.30 6.12 6.64 7.34, skinny 5.34 5.33 5.48 5.56, gemm 9.8-9.9
//   1.5B k/v 256 x 1536          dot 5.14 5.94 6.50 7.17, skinny 5.20 5.21 5.34 5.46, gemm 9.4
//   1.5B gate 8960 x 1536 (560)  dot 9.00 9.89 10.92 12.42, skinny 9.10 9.18 10.01 10.66, gemm 12.2-12.6
//   1.5B down 1536 x 8960 (96)   dot 10.65 11.81 13.20 15.39, skinny 17.0-18.3, gemm 13.25 13.39 13.55 14.04
//   1.5B gate_up 17920 x 1536 (1120)  dot 15.6 16.7 18.1 20.5, skinny 15.0 15.1 16.3 18.1, gemm 12.6-12.7
// and on >= 1024 tiles or long rows, M = 4..8 / 12..16:
//   1.5B gate_up 17920 x 1536 (1120 tiles), M = 4 5 6 7 8: skinny 11.67 12.19 13.94 14.49 15.02,
//                                            gemm 11.87 12.40 12.59 12.57 12.62
//   151936 x 896 (9496 tiles), M = 4 6 8 12 16: skinny 34.8 36.0 37.1 57.9 63.4, gemm 52.6 52.7 52.3 53.3 54.5
//   0.5B down 896 x 4864, M = 12 13 14 16: dot 9.42 9.77 10.17 10.77, skinny 10.6-11.0, gemm 11.4-11.5
//   1.5B down 1536 x 8960, M = 12 13 14 16: dot 13.21 13.72 14.44 15.30, gemm 13.31 13.35 13.35 13.42
// Then k_dot's MFMA path stored its plain epilogue in the MFMA layout (4
// outputs per lane of the tile's first wave instead of 2 M from one lane in
// eight), same graph replay, M = 3 / 8 / 9 / 12 / 16:
//   q 896 x 896                  dot 3.16 3.27 3.32 3.46 3.62, skinny 4.79 5.31 5.40 4.58 4.65
//   o 896 x 896                  dot 3.43 3.59 3.60 3.80 4.01, skinny 5.72 6.55 6.63 5.87 5.98
//   gate 4864 x 896              dot 3.98 4.17 4.24 4.47 4.78, skinny 5.61 6.23 6.32 5.85 6.09
//   gate_up 9728 x 896 (608)     dot 4.86 5.17 5.32 5.66 6.20, skinny 6.53 7.51 7.36 7.24 7.66, gemm 8.1-9.3
//   down 896 x 4864              dot 6.13 6.62 6.89 7.55 8.54, skinny 10.9-12.4, gemm 10.4-10.9
//   1.5B q/o 1536 x 1536         dot 3.82 4.08 4.15 4.35 4.65, skinny 5.66 5.28 5.30 5.43 5.55
//   1.5B k/v 256 x 1536          dot 3.66 3.94 4.01 4.24 4.49, skinny 5.50 5.15 5.16 5.32 5.40
//   1.5B gate 8960 x 1536 (560)  dot 6.68 7.56 7.83 8.48 9.43, skinny 8.36 9.07 9.15 9.96 10.70, gemm 10.4-10.9
//   1.5B down 1536 x 8960 (96)   dot 8.77 9.67 10.13 11.29 13.10, gemm 11.6-11.9, 12.23 at 16
//   1.5B gate_up 17920 x 1536 (1120)  dot 11.77 13.19 13.65 14.81 16.52, skinny 11.91 15.0 15.0 16.4 18.1,
//                                     gemm 12.5-12.8
// Then k_dot's MFMA path took the activation tile (whole-line activation
// loads regathered through LDS) in early launches re-reading >= 5 MB of
// activations with <= 12 k steps per wave, and the split-K reduction its
// split groups; same graph replay, M = 3 / 4 / 5 / 6 / 8 / 9 / 12 / 16:
//   1.5B gate_up 17920 x 1536 (1120)  dot 9.69 9.81 9.84 10.00 10.30 11.67 12.11 12.76,
//                                     skinny 11.88-17.86, gemm 12.50-12.83
//   151936 x 896 (9496 tiles)         dot 28.66 28.55 29.49 28.67 30.09 37.55 38.18 40.02,
//                                     skinny 34.2 35.2 35.8 36.2 37.4 37.4 57.6 63.0, gemm 53.6-55.9
//   1.5B down 1536 x 8960 (96)        dot 8.86 8.92 9.00 9.15 9.73 10.13 11.32 13.10,
//                                     gemm 10.36 10.40 10.43 10.39 10.75 10.37 10.57 11.37
//   (below 1024 tiles k_dot kept its lead at every M on every other shape)
// So: k_dot at M <= 2, and at M <= 8 below 1024 tiles; on 1024 and more
// tiles k_dot at M <= 16 where its launch takes the activation tile
// (dot_call_takes_x_tile); otherwise at M = 6..8 the GEMM when its 64 x 128
// tiles fit one round over the CUs; from M = 9, rows of at least kLongK
// codes on few tiles take k_dot up to M = 10 or M * K = 16 * 4864 and the
// split-K GEMM above, 1024 and more tiles (or rows of kGemmLongRows codes)
// the GEMM, the rest (short rows below 1024 tiles) k_dot's 16-row path;
// k_skinny for M <= 8 on 1024 and more tiles otherwise.  k_stream lost to
// k_skinny by 1.7-3.5x at every M and shape of the sweep (e.g. 151936 x 896:
// 58-78 us), so it runs only when forced.
constexpr std::size_t kDotAutoMaxM = 2;
constexpr std::size_t kDotAutoMfMaxM = 8;    // k_dot's MFMA path below kDotMfTiles tiles
constexpr std::size_t kDotLongMaxM = 10;     // M > 8: k_dot on long rows over few tiles up to this M,
constexpr int64_t kDotLongMaxMK = 16 * 4864; // or while M * K is at most this
constexpr std::size_t kGemmWideMinM = 6;     // M = 6..8 on >= kDotMfTiles tiles: the GEMM when its
                                             // 64 x 128 tiles fit one round over the CUs
constexpr int64_t kDotMfTiles = 1024;        // M = 3..16: below this many tiles k_dot / k_skinny, else
                                             // k_skinny (M <= 8) / the GEMM (M > 8)
constexpr int64_t kLongK = 4096;             // M > 8: long rows ...
constexpr int64_t kLongKMaxTiles = 128;      // ... on few 16-row tiles (N <= 2048)
constexpr std::size_t kSkinnyAutoMaxM = 8;
constexpr int64_t kGemmLongRows = 4096;      // M > 8: the GEMM on rows of this many codes over more tiles
// M = 17..64 (k_skinny with 2 or 4 groups of 16 rows against the GEMM, same
// graph replay), M = 17 / 32 / 48 / 64:
//   0.5B q/k/v 1152 x 896 (72 tiles)  skinny 5.46 6.27 8.38 9.64, gemm 9.94 9.98 10.16 10.41
//   0.5B o 896 x 896 (56)             skinny 5.45 6.24 8.31 9.58, gemm 9.89 9.91 10.10 10.33
//   1.5B q/o 1536 x 1536 (96)         skinny 6.79 7.68 10.31 12.05, gemm 10.01 10.09 10.57 10.90
//   1.5B k/v 256 x 1536 (16)          skinny 6.63 7.52 10.10 11.84, gemm 9.50 9.59 9.87 10.11
//   1.5B gate 8960 x 1536 (560)       skinny 12.06 16.0 20.95 25.49, gemm 12.68 13.53 14.88 11.89
//   0.5B down 896 x 4864 (56)         skinny 14.15 16.1 21.85 26.07, gemm 11.57 12.0 12.78 12.41
//   (gate/up and longer rows: the GEMM by 1.3-3.4x)
// so k_skinny at most kLongKMaxTiles tiles with M * K <= kSkinnyMgMaxMK.
constexpr int64_t kSkinnyMgMaxMK = 64 * 896;

int choose_ksplit(int64_t tiles, int64_t K, int64_t step);

// Whether a plain k_dot call with M > 2 rows takes the activation tile
// (launch_dot's choice for the call run_call makes, restated here).
bool dot_call_takes_x_tile(int64_t M, int64_t N, int64_t K)
{
    LinArgs a{};
    a.N = N;
    a.K = K;
    a.ksplit = choose_ksplit((N + kDecodeTileN - 1) / kDecodeTileN, K, kDotStep);
    // early plain calls load their activations with the weights (not in LDS)
    return dot_takes_x_tile(M, dot_early(dot_blocks(a)), false, dot_x_reread_bytes(M, N, K),
                            dot_wave_steps(K, a.ksplit));
}

int natural_kernel(std::size_t M, std::size_t N, std::size_t K, int act)
{
    if (act == VVH_F32) return (M >= kGemmF32MinM && K % kGemmBK == 0) ? K_GEMM : K_GEMV_F32;
    const int64_t tiles = ((int64_t)N + kDecodeTileN - 1) / kDecodeTileN;
    const bool dot_ok = dot_fits((int64_t)N, (int64_t)K);
    if ((M <= kDotAutoMaxM || (M <= kDotAutoMfMaxM && tiles < kDotMfTiles)) && dot_ok) return K_DOT;
    // 3-16 rows on many tiles: k_dot where its launch takes the activation tile
    if (M <= (std::size_t)kSkinnyMaxM && tiles >= kDotMfTiles && dot_ok &&
        dot_call_takes_x_tile((int64_t)M, (int64_t)N, (int64_t)K))
        return K_DOT;
    const int64_t cus = g_cu_count > 0 ? g_cu_count : 256;
    if (M >= kGemmWideMinM && M <= kSkinnyAutoMaxM && K % kGemmBK == 0 && ((int64_t)N + 127) / 128 <= cus)
        return K_GEMM;
    if (M > (std::size_t)kSkinnyMaxM) {
        // k_skinny with up to 4 groups of 16 rows: one weight pass, the
        // activations (M * K halves) read again by every wave, so few tiles
        // and short rows only
        if (M <= (std::size_t)kSkinnyMgMaxM && tiles <= kLongKMaxTiles && (int64_t)(M * K) <= kSkinnyMgMaxMK)
            return K_SKINNY;
        return K_GEMM;
    }
    if (M > kSkinnyAutoMaxM) {
        const bool gemm_ok = K % kGemmBK == 0;
        if ((int64_t)K >= kLongK && tiles <= kLongKMaxTiles) {
            if ((M <= kDotLongMaxM || (int64_t)(M * K) <= kDotLongMaxMK) && dot_ok) return K_DOT;
            if (gemm_ok) return K_GEMM;
        } else if (gemm_ok && (tiles >= kDotMfTiles || (int64_t)K >= kGemmLongRows)) {
            return K_GEMM;
        } else if (tiles < kDotMfTiles && dot_ok) {
            return K_DOT;
        }
    }
    return K_SKINNY;
}

// Kernel family for one call; `aligned` = K % 16 == 0 and 16-byte aligned
// weight and activation bases.  A family forced by vvh_set_kernel_override
// that cannot serve the call gives K_GENERIC.
int choose_kernel(std::size_t M, std::size_t N, std::size_t K, int act, bool aligned)
{
    if (K == 0 || !aligned) return K_GENERIC;
    const int ov = g_override.load();
    const int k = ov == K_AUTO ? natural_kernel(M, N, K, act) : ov;
    const bool decode = act == VVH_F16 && M <= (std::size_t)kSkinnyMaxM;
    switch (k) {
        case K_GEMV_F32: return act == VVH_F32 ? K_GEMV_F32 : K_GENERIC;
        case K_SKINNY: return (act == VVH_F16 && M <= (std::size_t)kSkinnyMgMaxM) ? K_SKINNY : K_GENERIC;
        case K_STREAM: return (decode && stream_depth(((int64_t)K + 63) / 64) > 0) ? K_STREAM : K_GENERIC;
        case K_DOT:
            return (act == VVH_F16 && M <= (std::size_t)kDotMaxM && dot_fits((int64_t)N, (int64_t)K)) ? K_DOT
                                                                                                        : K_GENERIC;
        case K_GEMM: return (act == VVH_F16 || K % kGemmBK == 0) ? K_GEMM : K_GENERIC;
        default: return K_GENERIC;
    }
}

// Waves of a block that split one tile's k range: enough waves in flight to
// cover every CU several times, never more than the k steps (of `step`
// codes) available.
int choose_ksplit(int64_t tiles, int64_t K, int64_t step = 64)
{
    const int64_t target = (int64_t)(g_cu_count > 0 ? g_cu_count : 256) * 8;
    int ks = tiles >= target ? 1 : (tiles * 2 >= target ? 2 : 4);
    const int64_t steps = (K + step - 1) / step;
    while (ks > 1 && ks > steps) ks >>= 1;
    return ks;
}

int validate_call(const void* out, const void* inp, const int8_t* w, const float* scales,
                  std::size_t M, std::size_t N, std::size_t K, int act, int outd)
{
    if (!valid_dtype(act) || !valid_dtype(outd))
        return fail(VVH_ERR_INVALID_ARG, "bad dtype (act %d, out %d)", act, outd);
    uint64_t mk, nk, mn;
    if (!mul_ok(M, K, &mk) || !mul_ok(N, K, &nk) || !mul_ok(M, N, &mn))
        return fail(VVH_ERR_INVALID_ARG, "size overflow (M %zu, N %zu, K %zu)", M, N, K);
    if (M == 0 || N == 0) return VVH_OK;
    if (!out) return fail(VVH_ERR_INVALID_ARG, "out is null");
    if (!scales) return fail(VVH_ERR_INVALID_ARG, "scales is null");
    if (K > 0 && (!inp || !w)) return fail(VVH_ERR_INVALID_ARG, "inp or weight is null");
    return VVH_OK;
}

int run_call(const LinArgs& base, int kernel, int act, int outd, void* stream, const WsSource* wsrc = nullptr)
{
    LinArgs a = base;
    int e = 0;
    switch (kernel) {
        case K_GEMV_F32: {
            a.ksplit = choose_ksplit((a.N + kDecodeTileN - 1) / kDecodeTileN, a.K);
            const int64_t mt = a.M <= 1 ? 1 : a.M <= 2 ? 2 : a.M <= 4 ? 4 : kGemvF32MaxM;
            if (decode_blocks(a) > INT32_MAX || (a.M + mt - 1) / mt > 65535)
                return fail(VVH_ERR_UNSUPPORTED, "problem too large for the decode grid");
            e = launch_gemv_f32(a, outd, stream);
            break;
        }
        case K_STREAM: {
            const int64_t tiles = (a.N + kDecodeTileN - 1) / kDecodeTileN;
            const int depth = stream_depth((a.K + 63) / 64);
            {
                StreamArgs sa{};
                sa.one = a;
                sa.total_tiles = tiles;
                sa.mode = kStreamRange;
                const int64_t per = (tiles + stream_max_waves() - 1) / stream_max_waves();
                const int64_t waves = (tiles + per - 1) / per;  // equal tile counts per wave
                sa.waves = (int32_t)waves;
                e = launch_stream(sa, depth, (int)a.M, outd, (waves + 3) / 4, stream);
            }
            break;
        }
        case K_DOT: {
            const int64_t tiles = (a.N + kDecodeTileN - 1) / kDecodeTileN;
            a.ksplit = choose_ksplit(tiles, a.K, kDotStep);
            if (a.ksplit == 4 && a.xop == 0 && dot_split8(a.M, tiles, a.K, g_cu_count > 0 ? g_cu_count : 256))
                a.ksplit = 8;
            if (dot_blocks(a) > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "problem too large for the decode grid");
            if (!dot_fits(a.N, a.K))
                return fail(VVH_ERR_UNSUPPORTED, "N (%lld) or K (%lld) too large for the decode kernel",
                            (long long)a.N, (long long)a.K);
            e = launch_dot(a, outd, dot_early(dot_blocks(a)), dot_depth(a.K, a.ksplit), stream);
            break;
        }
        case K_SKINNY: {
            const int64_t tiles = (a.N + kDecodeTileN - 1) / kDecodeTileN;
            a.ksplit = choose_ksplit(tiles, a.K);
            if (decode_blocks(a) > INT32_MAX)
                return fail(VVH_ERR_UNSUPPORTED, "problem too large for the decode grid");
            e = launch_skinny(a, outd, stream);
            break;
        }
        case K_GEMM: {
            const int64_t nb = ((a.M + kGemmBM - 1) / kGemmBM) * ((a.N + kGemmBN - 1) / kGemmBN);
            if (nb > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "problem too large for the GEMM grid");
            a.nsplit = 1;
            a.kstages = 0;
            a.ws = nullptr;
            if (a.K % kGemmBK == 0) {
                // fp32 activations: the GEMM runs on their split fp16 form
                // (M rows of 2K: scaled high parts, then low parts, plus one
                // inverse scale per row), made in the workspace first
                const bool f32 = act == VVH_F32;
                uint64_t xs_bytes = 0, rs_bytes = 0;
                if (f32) {
                    if (!mul_ok((uint64_t)a.M * (uint64_t)a.K, 4, &xs_bytes))
                        return fail(VVH_ERR_UNSUPPORTED, "problem too large for the fp32 GEMM path");
                    xs_bytes = align_up(xs_bytes);
                    rs_bytes = align_up((uint64_t)a.M * 4);
                }
                const int64_t stages = (f32 ? 2 * a.K : a.K) / kGemmBK;
                int split_layout = 4;
                int s = gemm_splits(a.M, a.N, stages, &split_layout);
                uint64_t plane = 0;
                if (s > 1) {
                    const int64_t kst = (stages + s - 1) / s;
                    s = (int)((stages + kst - 1) / kst);  // no empty split
                    if (s > 1 && mul_ok((uint64_t)a.M * (uint64_t)a.N, (uint64_t)s * 4, &plane) && nb * s <= INT32_MAX) {
                        a.nsplit = s;
                        a.kstages = (int32_t)kst;
                    } else {
                        plane = 0;
                    }
                }
                if (xs_bytes + rs_bytes + plane > 0) {
                    float* ws = nullptr;
                    const int st = workspace_get(wsrc, stream, xs_bytes + rs_bytes + plane, &ws);
                    if (st != VVH_OK) return st;
                    char* wb = reinterpret_cast<char*>(ws);
                    if (f32) {
                        e = launch_split_f32(static_cast<const float*>(a.inp), a.M, a.K, wb,
                                             reinterpret_cast<float*>(wb + xs_bytes), stream);
                        if (e != 0) break;
                        a.inp = wb;
                        a.xrs = reinterpret_cast<const float*>(wb + xs_bytes);
                        a.bk = a.K;
                        a.K = 2 * a.K;
                    }
                    if (a.nsplit > 1) a.ws = reinterpret_cast<float*>(wb + xs_bytes + rs_bytes);
                }
                {
                    const int layout = gemm3_layout(a.M, a.N, a.nsplit, split_layout);
                    const int64_t krange = a.nsplit > 1 ? (int64_t)a.kstages * kGemmBK : (a.bk ? a.bk : a.K);
                    const int64_t arow = a.nsplit > 1 ? (int64_t)a.kstages * kGemmBK : a.K;
                    a.norder = gemm3_norder(a.M, a.N, arow, krange, layout, a.nsplit);
                    e = launch_gemm3(a, outd, layout, stream);
                }
                if (e == 0 && a.nsplit > 1) e = launch_splitk_reduce(a, outd, stream);
                break;
            }
            e = launch_gemm(a, outd, stream);  // K % 64 != 0: never split
            break;
        }
        default: {
            if ((a.M * a.N + 255) / 256 > INT32_MAX)
                return fail(VVH_ERR_UNSUPPORTED, "problem too large for the generic kernel");
            e = launch_generic(a, act, outd, stream);
            break;
        }
    }
    if (e != 0) return fail_hip((hipError_t)e, "kernel launch");
    return VVH_OK;
}

// k_dot plan: problems ordered by K (longest rows first, so the last blocks
// dispatched are the short ones), each given its ksplit for the plan's total
// tile count and a contiguous range of blocks; a block -> problem map and
// the problem table go to the device in one allocation.
int build_dot_plan(Plan& p, int64_t total_tiles)
{
    std::stable_sort(p.args.begin(), p.args.end(), [](const LinArgs& x, const LinArgs& y) { return x.K > y.K; });
    int64_t blk = 0;
    int max_m = 0;
    size_t lds = 0;
    bool x_in_lds = true;
    for (const LinArgs& a : p.args) x_in_lds = x_in_lds && dot_x_in_lds(a.M, a.K);
    int depth = 2;
    for (LinArgs& a : p.args) {
        a.ksplit = choose_ksplit(total_tiles, a.K, kDotStep);
        depth = std::max(depth, dot_depth(a.K, a.ksplit));
        if (blk > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "plan too large");
        a.block_begin = (int32_t)blk;
        blk += dot_blocks(a);
        max_m = std::max(max_m, (int)a.M);
        lds = std::max(lds, (size_t)(x_in_lds ? dot_lds_bytes(a.M, a.K) : kDotRedBytes));
    }
    if (blk > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "plan too large");
    std::vector<int32_t> block_prob((size_t)blk);
    for (size_t i = 0; i < p.args.size(); i++) {
        const int64_t b0 = p.args[i].block_begin, b1 = b0 + dot_blocks(p.args[i]);
        for (int64_t b = b0; b < b1; b++) block_prob[(size_t)b] = (int32_t)i;
    }
    const size_t b_table = align_up(p.args.size() * sizeof(LinArgs));
    const size_t bytes = b_table + align_up((size_t)blk * 4);
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail_hip(e, "dot plan hipMalloc");
    }
    char* c = static_cast<char*>(base);
    if ((e = hipMemcpy(c, p.args.data(), p.args.size() * sizeof(LinArgs), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(c + b_table, block_prob.data(), (size_t)blk * 4, hipMemcpyHostToDevice)) != hipSuccess) {
        (void)hipFree(base);
        return fail_hip(e, "dot plan upload");
    }
    p.dot = true;
    p.dev_stream = base;  // owns table + map
    p.dev_table = nullptr;
    p.total_blocks = blk;
    p.max_m = max_m;
    p.dot_depth = depth;
    p.x_in_lds = x_in_lds;
    p.lds_bytes = lds;
    p.sargs = StreamArgs{};
    p.sargs.table = reinterpret_cast<const LinArgs*>(c);
    p.dev_block_prob = reinterpret_cast<int32_t*>(c + b_table);
    return VVH_OK;
}

// Streaming plan: problems ordered by K (longest rows first), their 16-row
// tiles numbered globally in that order, and each wave given a list of tiles
// by longest-processing-time-first assignment on weight bytes (each tile goes
// to the wave with the fewest bytes so far), so every wave streams about the
// same number of bytes.  One device allocation holds the problem table,
// the tile -> problem map, the per-wave lists and their offsets.
int build_stream_plan(Plan& p, int64_t total_tiles, int depth)
{
    if (total_tiles > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "plan too large for a streaming launch");
    std::stable_sort(p.args.begin(), p.args.end(), [](const LinArgs& x, const LinArgs& y) { return x.K > y.K; });
    const int64_t T = total_tiles;
    std::vector<int32_t> tile_prob((size_t)T);
    int64_t g = 0;
    for (size_t i = 0; i < p.args.size(); i++) {
        LinArgs& a = p.args[i];
        a.ksplit = 1;
        a.tile_begin = g;
        const int64_t n = (a.N + kDecodeTileN - 1) / kDecodeTileN;
        for (int64_t t = 0; t < n; t++) tile_prob[(size_t)(g + t)] = (int32_t)i;
        g += n;
    }
    const int64_t W = std::min<int64_t>(stream_max_waves(), T);
    // min-heap of (bytes, wave); tiles arrive in non-increasing size order
    std::vector<std::pair<int64_t, int32_t>> heap;
    heap.reserve((size_t)W);
    for (int64_t w = 0; w < W; w++) heap.emplace_back(0, (int32_t)w);
    std::vector<std::vector<int32_t>> lists((size_t)W);
    auto cmp = [](const std::pair<int64_t, int32_t>& x, const std::pair<int64_t, int32_t>& y) { return x > y; };
    for (int64_t t = 0; t < T; t++) {
        std::pop_heap(heap.begin(), heap.end(), cmp);
        auto& top = heap.back();
        lists[(size_t)top.second].push_back((int32_t)t);
        top.first += kDecodeTileN * p.args[(size_t)tile_prob[(size_t)t]].K;
        std::push_heap(heap.begin(), heap.end(), cmp);
    }
    std::vector<int32_t> list, off;
    list.reserve((size_t)T);
    off.reserve((size_t)W + 1);
    for (auto& l : lists) {
        off.push_back((int32_t)list.size());
        list.insert(list.end(), l.begin(), l.end());
    }
    off.push_back((int32_t)list.size());

    const size_t b_table = align_up(p.args.size() * sizeof(LinArgs));
    const size_t b_prob = align_up((size_t)T * 4), b_list = align_up((size_t)T * 4);
    const size_t bytes = b_table + b_prob + b_list + align_up(off.size() * 4);
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail_hip(e, "stream plan hipMalloc");
    }
    char* c = static_cast<char*>(base);
    if ((e = hipMemcpy(c, p.args.data(), p.args.size() * sizeof(LinArgs), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(c + b_table, tile_prob.data(), (size_t)T * 4, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(c + b_table + b_prob, list.data(), (size_t)T * 4, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(c + b_table + b_prob + b_list, off.data(), off.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) {
        (void)hipFree(base);
        return fail_hip(e, "stream plan upload");
    }
    p.stream = true;
    p.depth = depth;
    p.max_m = 0;
    for (const LinArgs& a : p.args) p.max_m = std::max(p.max_m, (int)a.M);
    p.dev_stream = base;
    StreamArgs& sa = p.sargs;
    sa = StreamArgs{};
    sa.table = reinterpret_cast<const LinArgs*>(c);
    sa.tile_prob = reinterpret_cast<const int32_t*>(c + b_table);
    sa.list = reinterpret_cast<const int32_t*>(c + b_table + b_prob);
    sa.list_off = reinterpret_cast<const int32_t*>(c + b_table + b_prob + b_list);
    sa.total_tiles = T;
    sa.waves = (int32_t)W;
    sa.mode = kStreamList;
    return VVH_OK;
}

}  // namespace

int vvh::linear_dev(void* out, const void* inp, const int8_t* w, const float* scales, const float* bias,
               const void* res, std::size_t M, std::size_t N, std::size_t K, int act, int outd,
               void* stream, const WsSource* wsrc)
{
    int st = validate_call(out, inp, w, scales, M, N, K, act, outd);
    if (st != VVH_OK || M == 0 || N == 0) return st;
    REQUIRE_INIT();
    LinArgs a{};
    a.out = out;
    a.inp = inp;
    a.res = res;
    a.w = w;
    a.scales = scales;
    a.bias = bias;
    a.M = (int64_t)M;
    a.N = (int64_t)N;
    a.K = (int64_t)K;
    a.ksplit = 1;
    const bool aligned = K % 16 == 0 && aligned16(w) && aligned16(inp);
    return run_call(a, choose_kernel(M, N, K, act, aligned), act, outd, stream, wsrc);
}

extern "C" {

VVH_API const char* vvh_status_string(int status)
{
    switch (status) {
        case VVH_OK: return "VVH_OK";
        case VVH_ERR_INVALID_ARG: return "VVH_ERR_INVALID_ARG";
        case VVH_ERR_NO_DEVICE: return "VVH_ERR_NO_DEVICE";
        case VVH_ERR_OUT_OF_MEMORY: return "VVH_ERR_OUT_OF_MEMORY";
        case VVH_ERR_HIP: return "VVH_ERR_HIP";
        case VVH_ERR_NOT_INITIALIZED: return "VVH_ERR_NOT_INITIALIZED";
        case VVH_ERR_UNKNOWN_HANDLE: return "VVH_ERR_UNKNOWN_HANDLE";
        case VVH_ERR_UNSUPPORTED: return "VVH_ERR_UNSUPPORTED";
        default: return "VVH_ERR_UNKNOWN_STATUS";
    }
}

VVH_API const char* vvh_last_error(void) { return g_last_error.c_str(); }

VVH_API const char* vvh_version(void) { return "vvllm-hip 0.1 gfx950"; }

VVH_API int vvh_init(int device, char* name_buf, size_t name_buf_size)
{
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return fail(VVH_ERR_NO_DEVICE, "no HIP device (%s)", hipGetErrorString(e));
    }
    if (device < 0 || device >= count)
        return fail(VVH_ERR_NO_DEVICE, "device %d out of range [0, %d)", device, count);
    if ((e = hipSetDevice(device)) != hipSuccess) return fail_hip(e, "hipSetDevice");
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
        return fail_hip(e, "hipGetDeviceProperties");
    const int st = scratch_setup(device);
    if (st != VVH_OK) return st;
    g_device = device;
    g_cu_count = prop.multiProcessorCount;
    if (name_buf && name_buf_size > 0) {
        snprintf(name_buf, name_buf_size, "%s (%s, %d CUs)", prop.name[0] ? prop.name : "AMD GPU",
                 prop.gcnArchName, prop.multiProcessorCount);
    }
    g_init.store(true);
    return VVH_OK;
}

VVH_API int vvh_sync(void)
{
    REQUIRE_INIT();
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? VVH_OK : fail_hip(e, "hipDeviceSynchronize");
}

VVH_API int vvh_device_cu_count(void) { return g_init.load() ? g_cu_count : 0; }

// ---- raw memory ---------------------------------------------------------------
VVH_API int vvh_malloc(void** ptr, size_t bytes)
{
    if (!ptr) return fail(VVH_ERR_INVALID_ARG, "ptr is null");
    *ptr = nullptr;
    REQUIRE_INIT();
    if (bytes == 0) return VVH_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *ptr = nullptr;
        return fail_hip(e, "hipMalloc");
    }
    return VVH_OK;
}

VVH_API int vvh_free(void* ptr)
{
    if (!ptr) return VVH_OK;
    REQUIRE_INIT();
    hipError_t e = hipFree(ptr);
    return e == hipSuccess ? VVH_OK : fail_hip(e, "hipFree");
}

VVH_API int vvh_malloc_host(void** ptr, size_t bytes)
{
    if (!ptr) return fail(VVH_ERR_INVALID_ARG, "ptr is null");
    *ptr = nullptr;
    REQUIRE_INIT();
    if (bytes == 0) return VVH_OK;
    hipError_t e = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *ptr = nullptr;
        return fail_hip(e, "hipHostMalloc");
    }
    return VVH_OK;
}

VVH_API int vvh_free_host(void* ptr)
{
    if (!ptr) return VVH_OK;
    REQUIRE_INIT();
    hipError_t e = hipHostFree(ptr);
    return e == hipSuccess ? VVH_OK : fail_hip(e, "hipHostFree");
}

static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, const char* what)
{
    if (bytes == 0) return VVH_OK;
    if (!dst || !src) return fail(VVH_ERR_INVALID_ARG, "%s: null pointer", what);
    REQUIRE_INIT();
    hipError_t e = hipMemcpy(dst, src, bytes, kind);
    return e == hipSuccess ? VVH_OK : fail_hip(e, what);
}

VVH_API int vvh_memcpy_h2d(void* d, const void* s, size_t n) { return copy(d, s, n, hipMemcpyHostToDevice, "memcpy h2d"); }
VVH_API int vvh_memcpy_d2h(void* d, const void* s, size_t n) { return copy(d, s, n, hipMemcpyDeviceToHost, "memcpy d2h"); }
VVH_API int vvh_memcpy_d2d(void* d, const void* s, size_t n) { return copy(d, s, n, hipMemcpyDeviceToDevice, "memcpy d2d"); }

VVH_API int vvh_memcpy_d2d_async(void* d, const void* s, size_t n, void* stream)
{
    if (n == 0) return VVH_OK;
    if (!d || !s) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    REQUIRE_INIT();
    const hipError_t e = hipMemcpyAsync(d, s, n, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VVH_OK : fail_hip(e, "memcpy d2d async");
}

// ---- caching allocator -------------------------------------------------------------
VVH_API int vvh_pool_alloc(void** ptr, size_t bytes)
{
    if (!ptr) return fail(VVH_ERR_INVALID_ARG, "ptr is null");
    *ptr = nullptr;
    REQUIRE_INIT();
    const int rc = g_pool.alloc(ptr, bytes);
    if (rc == 0) return VVH_OK;
    if (rc == 1) return fail(VVH_ERR_OUT_OF_MEMORY, "pool: out of device memory for %zu bytes", bytes);
    if (rc == 3) return fail(VVH_ERR_INVALID_ARG, "pool: size %zu too large", bytes);
    return fail(VVH_ERR_HIP, "pool: hipMalloc failed for %zu bytes", bytes);
}

VVH_API int vvh_pool_free(void* ptr)
{
    if (!ptr) return VVH_OK;
    REQUIRE_INIT();
    if (g_pool.free(ptr) == 0) return VVH_OK;
    hipError_t e = hipFree(ptr);  // not from the pool: a real free (tensor.cc:58-66)
    return e == hipSuccess ? VVH_OK : fail_hip(e, "hipFree");
}

VVH_API int vvh_pool_release_cached(void)
{
    REQUIRE_INIT();
    const int failures = g_pool.release_cached();
    return failures == 0 ? VVH_OK : fail(VVH_ERR_HIP, "pool: %d hipFree calls failed", failures);
}

VVH_API int vvh_pool_get_stats(vvh_pool_stats* out)
{
    if (!out) return fail(VVH_ERR_INVALID_ARG, "out is null");
    const PoolStats s = g_pool.stats();
    out->bytes_in_use = s.bytes_in_use;
    out->bytes_cached = s.bytes_cached;
    out->bytes_reserved = s.bytes_in_use + s.bytes_cached;
    out->peak_reserved = s.peak_reserved;
    out->alloc_calls = s.alloc_calls;
    out->cache_hits = s.cache_hits;
    out->driver_allocs = s.driver_allocs;
    out->oom_releases = s.oom_releases;
    return VVH_OK;
}

// ---- weight mirror ---------------------------------------------------------------
static void drop_weight_locked(vvh_weight h)
{
    auto it = g_weights.find(h);
    if (it == g_weights.end()) return;
    if (it->second.base) (void)hipFree(it->second.base);
    if (it->second.host_w) {
        auto hb = g_weight_by_host.find(it->second.host_w);
        if (hb != g_weight_by_host.end() && hb->second == h) g_weight_by_host.erase(hb);
    }
    g_weights.erase(it);
}

VVH_API int vvh_weight_register(const int8_t* host_weight, const float* host_scales,
                                const float* host_bias, size_t N, size_t K, vvh_weight* handle)
{
    if (!handle) return fail(VVH_ERR_INVALID_ARG, "handle is null");
    *handle = 0;
    if (!host_weight || !host_scales) return fail(VVH_ERR_INVALID_ARG, "weight or scales is null");
    uint64_t nk;
    if (N == 0 || !mul_ok(N, K, &nk)) return fail(VVH_ERR_INVALID_ARG, "bad shape N %zu K %zu", N, K);
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_wmu);
    auto hb = g_weight_by_host.find(host_weight);
    if (hb != g_weight_by_host.end()) {
        const WeightEntry& e = g_weights.at(hb->second);
        if (e.host_scales == host_scales && e.host_bias == host_bias && e.N == N && e.K == K) {
            *handle = hb->second;  // also an ingested mirror: its codes came from these rows
            return VVH_OK;
        }
        drop_weight_locked(hb->second);  // same host buffer, new contents/shape
    }
    const std::size_t off_s = align_up(nk);
    const std::size_t off_b = off_s + align_up(N * sizeof(float));
    const std::size_t bytes = off_b + (host_bias ? align_up(N * sizeof(float)) : 0);
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (g_pool.release_cached() == 0 && hipMalloc(&base, bytes) == hipSuccess) {
            e = hipSuccess;
        } else {
            (void)hipGetLastError();
            return fail_hip(e, "weight mirror hipMalloc");
        }
    }
    char* b = static_cast<char*>(base);
    if ((nk && (e = hipMemcpy(b, host_weight, nk, hipMemcpyHostToDevice)) != hipSuccess) ||
        (e = hipMemcpy(b + off_s, host_scales, N * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess ||
        (host_bias && (e = hipMemcpy(b + off_b, host_bias, N * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess)) {
        (void)hipFree(base);
        return fail_hip(e, "weight mirror upload");
    }
    WeightEntry w;
    w.host_w = host_weight;
    w.host_scales = host_scales;
    w.host_bias = host_bias;
    w.N = N;
    w.K = K;
    w.base = base;
    w.bytes = bytes;
    w.w = reinterpret_cast<const int8_t*>(b);
    w.scales = reinterpret_cast<const float*>(b + off_s);
    w.bias = host_bias ? reinterpret_cast<const float*>(b + off_b) : nullptr;
    const vvh_weight h = g_next_weight++;
    g_weights.emplace(h, w);
    g_weight_by_host[host_weight] = h;
    *handle = h;
    return VVH_OK;
}

// Weight ingestion: host rows of F32 or BF16 go to the device in their stored
// width through two pinned staging buffers (the CPU fills one while the DMA
// engine drains the other), are widened in registers and quantized into the
// new mirror.  The reference widens BF16 to fp32 on the host
// (src/safetensors/safetensors.cc:112-119) and quantizes on the host
// (src/model/qwen2/model.cc:27-33, src/quantize/quantize.cc:9-48).
namespace {
constexpr std::size_t kIngestChunk = std::size_t(32) << 20;  // bytes of source rows per chunk

// Staging of vvh_weight_ingest, allocated on first use and kept (pinning
// host memory costs milliseconds); used under g_wmu.  A row longer than the
// chunk grows it.
struct IngestStaging {
    void* host[2] = {nullptr, nullptr};
    void* dev[2] = {nullptr, nullptr};
    hipEvent_t copied[2] = {nullptr, nullptr};
    hipStream_t stream = nullptr;
    std::size_t bytes = 0;

    void release()
    {
        if (stream) (void)hipStreamSynchronize(stream);
        for (int i = 0; i < 2; i++) {
            if (host[i]) (void)hipHostFree(host[i]);
            if (dev[i]) (void)hipFree(dev[i]);
            host[i] = dev[i] = nullptr;
        }
        bytes = 0;
    }
    hipError_t ensure(std::size_t need)
    {
        hipError_t e = hipSuccess;
        if (!stream && (e = hipStreamCreate(&stream)) != hipSuccess) return e;
        for (int i = 0; i < 2; i++)
            if (!copied[i] && (e = hipEventCreateWithFlags(&copied[i], hipEventDisableTiming)) != hipSuccess) return e;
        if (bytes >= need) return hipSuccess;
        release();
        for (int i = 0; i < 2; i++) {
            if ((e = hipHostMalloc(&host[i], need, hipHostMallocDefault)) != hipSuccess ||
                (e = hipMalloc(&dev[i], need)) != hipSuccess) {
                release();
                return e;
            }
        }
        bytes = need;
        return hipSuccess;
    }
};
IngestStaging g_ingest;
}  // namespace

VVH_API int vvh_weight_ingest(const void* host_weight, int src_dtype, const float* host_bias, size_t N, size_t K,
                              float* host_scales, vvh_weight* handle)
{
    if (!handle) return fail(VVH_ERR_INVALID_ARG, "handle is null");
    *handle = 0;
    if (src_dtype != VVH_F32 && src_dtype != VVH_BF16) return fail(VVH_ERR_INVALID_ARG, "bad source dtype %d", src_dtype);
    if (!host_weight || !host_scales) return fail(VVH_ERR_INVALID_ARG, "weight or scales is null");
    const std::size_t es = src_dtype == VVH_BF16 ? 2 : 4;
    uint64_t nk, src_bytes;
    if (N == 0 || K == 0 || !mul_ok(N, K, &nk) || !mul_ok(nk, es, &src_bytes))
        return fail(VVH_ERR_INVALID_ARG, "bad shape N %zu K %zu", N, K);
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_wmu);
    auto hb = g_weight_by_host.find(host_weight);
    if (hb != g_weight_by_host.end()) {
        const WeightEntry& e = g_weights.at(hb->second);
        if (e.host_scales == host_scales && e.host_bias == host_bias && e.N == N && e.K == K &&
            e.src_dtype == src_dtype) {
            *handle = hb->second;
            return VVH_OK;
        }
        drop_weight_locked(hb->second);
    }
    const std::size_t off_s = align_up(nk);
    const std::size_t off_b = off_s + align_up(N * sizeof(float));
    const std::size_t bytes = off_b + (host_bias ? align_up(N * sizeof(float)) : 0);
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (g_pool.release_cached() == 0 && hipMalloc(&base, bytes) == hipSuccess) {
            e = hipSuccess;
        } else {
            (void)hipGetLastError();
            return fail_hip(e, "weight mirror hipMalloc");
        }
    }
    char* b = static_cast<char*>(base);
    int8_t* codes = reinterpret_cast<int8_t*>(b);
    float* scales = reinterpret_cast<float*>(b + off_s);
    const std::size_t row_bytes = K * es;
    const std::size_t rows_per = std::max<std::size_t>(1, std::min<std::size_t>(N, kIngestChunk / row_bytes));
    const std::size_t chunk = rows_per * row_bytes;
    {
        IngestStaging& st = g_ingest;
        auto bail = [&](hipError_t err, const char* what) {
            (void)hipGetLastError();
            (void)hipFree(base);
            return fail_hip(err, what);
        };
        if ((e = st.ensure(std::max(chunk, kIngestChunk))) != hipSuccess) return bail(e, "ingest: staging");
        const char* src = static_cast<const char*>(host_weight);
        int c = 0;
        for (std::size_t r0 = 0; r0 < N; r0 += rows_per, c ^= 1) {
            const std::size_t rows = std::min(rows_per, N - r0);
            // the copy that last read this pinned buffer must be done
            if ((e = hipEventSynchronize(st.copied[c])) != hipSuccess) return bail(e, "ingest: wait");
            std::memcpy(st.host[c], src + r0 * row_bytes, rows * row_bytes);
            int k = 0;
            if ((e = hipMemcpyAsync(st.dev[c], st.host[c], rows * row_bytes, hipMemcpyHostToDevice, st.stream)) !=
                    hipSuccess ||
                (e = hipEventRecord(st.copied[c], st.stream)) != hipSuccess ||
                (k = launch_quantize(st.dev[c], src_dtype, (int64_t)rows, (int64_t)K, codes + r0 * K, scales + r0,
                                     st.stream)) != 0)
                return bail(k ? (hipError_t)k : e, "ingest: copy / quantize");
        }
        if ((e = hipStreamSynchronize(st.stream)) != hipSuccess ||
            (e = hipMemcpy(host_scales, scales, N * sizeof(float), hipMemcpyDeviceToHost)) != hipSuccess ||
            (host_bias && (e = hipMemcpy(b + off_b, host_bias, N * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess))
            return bail(e, "ingest: finish");
    }
    WeightEntry w;
    w.host_w = host_weight;
    w.host_scales = host_scales;
    w.host_bias = host_bias;
    w.N = N;
    w.K = K;
    w.src_dtype = src_dtype;
    w.base = base;
    w.bytes = bytes;
    w.w = codes;
    w.scales = scales;
    w.bias = host_bias ? reinterpret_cast<const float*>(b + off_b) : nullptr;
    const vvh_weight h = g_next_weight++;
    g_weights.emplace(h, w);
    g_weight_by_host[host_weight] = h;
    *handle = h;
    return VVH_OK;
}

VVH_API int vvh_weight_register_device(const int8_t* dev_weight, const float* dev_scales,
                                       const float* dev_bias, size_t N, size_t K, vvh_weight* handle)
{
    if (!handle) return fail(VVH_ERR_INVALID_ARG, "handle is null");
    *handle = 0;
    uint64_t nk;
    if ((K > 0 && !dev_weight) || !dev_scales) return fail(VVH_ERR_INVALID_ARG, "weight or scales is null");
    if (N == 0 || !mul_ok(N, K, &nk)) return fail(VVH_ERR_INVALID_ARG, "bad shape N %zu K %zu", N, K);
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_wmu);
    WeightEntry w;
    w.N = N;
    w.K = K;
    w.w = dev_weight;
    w.scales = dev_scales;
    w.bias = dev_bias;
    const vvh_weight h = g_next_weight++;
    g_weights.emplace(h, w);
    *handle = h;
    return VVH_OK;
}

VVH_API int vvh_weight_find(const int8_t* host_weight, vvh_weight* handle)
{
    if (!handle) return fail(VVH_ERR_INVALID_ARG, "handle is null");
    *handle = 0;
    std::lock_guard<std::mutex> lock(g_wmu);
    auto hb = g_weight_by_host.find(host_weight);
    if (hb == g_weight_by_host.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "host weight not mirrored");
    *handle = hb->second;
    return VVH_OK;
}

VVH_API int vvh_weight_release(vvh_weight handle)
{
    std::lock_guard<std::mutex> lock(g_wmu);
    if (!g_weights.count(handle)) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown weight handle %llu", (unsigned long long)handle);
    drop_weight_locked(handle);
    return VVH_OK;
}

VVH_API int vvh_weight_device_ptrs(vvh_weight handle, const int8_t** dev_weight, const float** dev_scales,
                                   const float** dev_bias, size_t* N, size_t* K)
{
    std::lock_guard<std::mutex> lock(g_wmu);
    auto it = g_weights.find(handle);
    if (it == g_weights.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown weight handle %llu", (unsigned long long)handle);
    if (dev_weight) *dev_weight = it->second.w;
    if (dev_scales) *dev_scales = it->second.scales;
    if (dev_bias) *dev_bias = it->second.bias;
    if (N) *N = it->second.N;
    if (K) *K = it->second.K;
    return VVH_OK;
}

VVH_API int vvh_weight_stats(uint64_t* count, uint64_t* bytes)
{
    std::lock_guard<std::mutex> lock(g_wmu);
    uint64_t b = 0;
    for (auto& kv : g_weights) b += kv.second.bytes;
    if (count) *count = g_weights.size();
    if (bytes) *bytes = b;
    return VVH_OK;
}

// ---- linear -----------------------------------------------------------------------
VVH_API int vvh_linear_q8_dev(void* out, const void* inp, const int8_t* dev_weight, const float* dev_scales,
                              const float* dev_bias, const void* residual, size_t M, size_t N, size_t K,
                              int act_dtype, int out_dtype, void* stream)
{
    return linear_dev(out, inp, dev_weight, dev_scales, dev_bias, residual, M, N, K, act_dtype, out_dtype, stream,
                      nullptr);
}

VVH_API int vvh_linear_q8_dev_noalloc(void* out, const void* inp, const int8_t* dev_weight,
                                      const float* dev_scales, const float* dev_bias, const void* residual,
                                      size_t M, size_t N, size_t K, int act_dtype, int out_dtype, void* stream)
{
    REQUIRE_INIT();
    void* scratch = g_device >= 0 && g_device < kMaxDevices ? g_scratch_ptr[g_device] : nullptr;
    if (!scratch)
        return fail(VVH_ERR_UNSUPPORTED, "no fixed scratch on device %d (devices 0..%d have one)", g_device,
                    kMaxDevices - 1);
    const WsSource src{scratch, VVH_NOALLOC_SCRATCH_BYTES};
    return linear_dev(out, inp, dev_weight, dev_scales, dev_bias, residual, M, N, K, act_dtype, out_dtype, stream,
                      &src);
}

VVH_API int vvh_workspace_release(void* stream)
{
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_wsmu);
    auto it = g_ws.find(stream);
    if (it == g_ws.end()) return VVH_OK;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail_hip(e, "workspace release: synchronize");
    for (void* p : it->second.retired) (void)hipFree(p);
    if (it->second.p) (void)hipFree(it->second.p);
    if (it->second.cnt) (void)hipFree(it->second.cnt);
    g_ws.erase(it);
    return VVH_OK;
}

// The input stage runs in k_dot's activation staging only: fp16 activations,
// M <= kStageMaxM, K % 16 == 0, aligned operands and the rows in LDS.
static int input_op_ok(int in_op, const float* in_w, std::size_t M, std::size_t K, int act)
{
    if (in_op < VVH_IN_NONE || in_op > VVH_IN_SILU_MUL) return fail(VVH_ERR_INVALID_ARG, "bad input op %d", in_op);
    if (in_op == VVH_IN_NONE) return VVH_OK;
    if (in_op == VVH_IN_RMS_NORM && (!in_w || !aligned16(in_w)))
        return fail(VVH_ERR_INVALID_ARG, "RMSNorm input stage needs 16-byte aligned weights");
    if (act != VVH_F16 || M == 0 || M > (std::size_t)kStageMaxM || K % 16 != 0 ||
        !dot_x_in_lds((int64_t)M, (int64_t)K))
        return fail(VVH_ERR_UNSUPPORTED, "input stage needs fp16 activations, M <= %d, K %% 16 == 0 and "
                    "rows that fit the block's LDS (M=%zu, K=%zu)", kStageMaxM, M, K);
    return VVH_OK;
}

VVH_API int vvh_linear_q8_dev_in(void* out, const void* inp, const int8_t* dev_weight, const float* dev_scales,
                                 const float* dev_bias, const void* residual, size_t M, size_t N, size_t K,
                                 int act_dtype, int out_dtype, int in_op, const float* in_w, float in_eps,
                                 void* stream)
{
    if (in_op == VVH_IN_NONE)
        return linear_dev(out, inp, dev_weight, dev_scales, dev_bias, residual, M, N, K, act_dtype, out_dtype, stream,
                          nullptr);
    int st = validate_call(out, inp, dev_weight, dev_scales, M, N, K, act_dtype, out_dtype);
    if (st != VVH_OK) return st;
    if ((st = input_op_ok(in_op, in_w, M, K, act_dtype)) != VVH_OK) return st;
    if (N == 0) return VVH_OK;
    REQUIRE_INIT();
    if (!aligned16(dev_weight) || !aligned16(inp))
        return fail(VVH_ERR_UNSUPPORTED, "input stage needs 16-byte aligned weights and activations");
    LinArgs a{};
    a.out = out;
    a.inp = inp;
    a.res = residual;
    a.w = dev_weight;
    a.scales = dev_scales;
    a.bias = dev_bias;
    a.M = (int64_t)M;
    a.N = (int64_t)N;
    a.K = (int64_t)K;
    a.ksplit = 1;
    a.xop = in_op;
    a.xw = in_w;
    a.xeps = in_eps;
    return run_call(a, K_DOT, act_dtype, out_dtype, stream);
}

VVH_API int vvh_linear_q8_dev_attn(void* out, const float* parts, size_t nparts, size_t head_dim,
                                   const int8_t* dev_weight, const float* dev_scales, const float* dev_bias,
                                   const void* residual, size_t N, size_t K, int out_dtype, void* stream)
{
    int st = validate_call(out, parts, dev_weight, dev_scales, 1, N, K, VVH_F16, out_dtype);
    if (st != VVH_OK) return st;
    if (nparts == 0 || nparts > (std::size_t)kAttnMaxParts)
        return fail(VVH_ERR_INVALID_ARG, "nparts %zu outside 1..%d", nparts, kAttnMaxParts);
    if (head_dim < 4 || head_dim > (std::size_t)kAttnMergeMaxK || (head_dim & (head_dim - 1)) != 0 ||
        K % head_dim != 0)
        return fail(VVH_ERR_INVALID_ARG, "K (%zu) must be a multiple of head_dim (%zu), a power of two from 4",
                    K, head_dim);
    if (K % 16 != 0 || K > (std::size_t)kAttnMergeMaxK || !dot_x_in_lds(1, (int64_t)K))
        return fail(VVH_ERR_UNSUPPORTED, "attention merge stage needs K %% 16 == 0 and K <= %d (K=%zu)",
                    (int)kAttnMergeMaxK, K);
    if (N == 0) return VVH_OK;
    REQUIRE_INIT();
    if (!aligned16(dev_weight) || !aligned16(parts))
        return fail(VVH_ERR_UNSUPPORTED, "attention merge stage needs 16-byte aligned weights and parts");
    LinArgs a{};
    a.out = out;
    a.inp = parts;
    a.res = residual;
    a.w = dev_weight;
    a.scales = dev_scales;
    a.bias = dev_bias;
    a.M = 1;
    a.N = (int64_t)N;
    a.K = (int64_t)K;
    a.ksplit = 1;
    a.xop = 3;
    a.xparts = (int32_t)nparts;
    a.xhd = (int32_t)head_dim;
    return run_call(a, K_DOT, VVH_F16, out_dtype, stream);
}

VVH_API int vvh_linear_q8(void* out, const void* inp, vvh_weight weight, const void* residual, size_t M,
                          size_t N, size_t K, int act_dtype, int out_dtype, void* stream)
{
    REQUIRE_INIT();
    const int8_t* w;
    const float *s, *b;
    {
        std::lock_guard<std::mutex> lock(g_wmu);
        auto it = g_weights.find(weight);
        if (it == g_weights.end())
            return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown weight handle %llu", (unsigned long long)weight);
        if (it->second.N != N || it->second.K != K)
            return fail(VVH_ERR_INVALID_ARG, "weight is [%zu, %zu], call asks for [%zu, %zu]", it->second.N,
                        it->second.K, N, K);
        w = it->second.w;
        s = it->second.scales;
        b = it->second.bias;
    }
    return linear_dev(out, inp, w, s, b, residual, M, N, K, act_dtype, out_dtype, stream, nullptr);
}

// ---- plans --------------------------------------------------------------------------
VVH_API int vvh_plan_create(const vvh_q8_problem* problems, size_t count, int act_dtype, int out_dtype,
                            vvh_plan* plan)
{
    if (!plan) return fail(VVH_ERR_INVALID_ARG, "plan is null");
    *plan = 0;
    if (!problems || count == 0) return fail(VVH_ERR_INVALID_ARG, "empty problem list");
    if (count > (size_t)INT32_MAX) return fail(VVH_ERR_INVALID_ARG, "too many problems");
    Plan p;
    p.act = act_dtype;
    p.out = out_dtype;
    bool all_skinny = true;  // every problem takes a decode kernel (M <= 16)
    bool all_dot = true;     // every problem takes k_dot (M <= 2)
    int64_t total_tiles = 0;
    for (size_t i = 0; i < count; i++) {
        const vvh_q8_problem& q = problems[i];
        int st = validate_call(q.out, q.inp, q.weight, q.scales, q.M, q.N, q.K, act_dtype, out_dtype);
        if (st != VVH_OK) return fail(st, "problem %zu: %s", i, vvh_last_error());
        if (q.M == 0 || q.N == 0) continue;
        LinArgs a{};
        a.out = q.out;
        a.inp = q.inp;
        a.res = q.residual;
        a.w = q.weight;
        a.scales = q.scales;
        a.bias = q.bias;
        a.M = (int64_t)q.M;
        a.N = (int64_t)q.N;
        a.K = (int64_t)q.K;
        a.ksplit = 1;
        a.src = (int32_t)i;
        const bool aligned = q.K % 16 == 0 && aligned16(q.weight) && aligned16(q.inp);
        const int kf = choose_kernel(q.M, q.N, q.K, act_dtype, aligned);
        // the grouped decode launches take one 16-row activation group
        if ((kf != K_SKINNY && kf != K_STREAM && kf != K_DOT) || (kf == K_SKINNY && q.M > (std::size_t)kSkinnyMaxM))
            all_skinny = false;
        if (kf != K_DOT) all_dot = false;
        total_tiles += (a.N + kDecodeTileN - 1) / kDecodeTileN;
        p.args.push_back(a);
    }
    if (p.args.empty()) return fail(VVH_ERR_INVALID_ARG, "every problem is empty");
    REQUIRE_INIT();
    int64_t min_steps = INT64_MAX;
    for (const LinArgs& a : p.args) min_steps = std::min(min_steps, (a.K + 63) / 64);
    // every problem takes a decode kernel: one k_skinny_grouped launch, or
    // one streaming launch when that family is forced
    const int ov = g_override.load();
    const int depth = all_skinny && ov != K_SKINNY ? stream_depth(min_steps) : 0;
    if (all_dot && (ov == K_AUTO || ov == K_DOT)) {
        const int st = build_dot_plan(p, total_tiles);
        if (st != VVH_OK) return st;
    } else if (depth > 0 && ov == K_STREAM) {
        const int st = build_stream_plan(p, total_tiles, depth);
        if (st != VVH_OK) return st;
    } else if (all_skinny) {
        p.grouped = true;
        // longest rows first, so the last blocks dispatched are the short ones
        std::stable_sort(p.args.begin(), p.args.end(),
                         [](const LinArgs& x, const LinArgs& y) { return x.K > y.K; });
        int64_t blk = 0;
        for (LinArgs& a : p.args) {
            a.ksplit = choose_ksplit(total_tiles, a.K);
            if (blk > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "plan too large");
            a.block_begin = (int32_t)blk;
            blk += decode_blocks(a);
        }
        if (blk > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "plan too large");
        p.total_blocks = blk;
        const size_t bytes = p.args.size() * sizeof(LinArgs);
        hipError_t e = hipMalloc(reinterpret_cast<void**>(&p.dev_table), bytes);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail_hip(e, "plan table hipMalloc");
        }
        if ((e = hipMemcpy(p.dev_table, p.args.data(), bytes, hipMemcpyHostToDevice)) != hipSuccess) {
            (void)hipFree(p.dev_table);
            return fail_hip(e, "plan table upload");
        }
    }
    std::lock_guard<std::mutex> lock(g_pmu);
    const vvh_plan h = g_next_plan++;
    g_plans.emplace(h, std::move(p));
    *plan = h;
    return VVH_OK;
}

static int plan_run(vvh_plan plan, int64_t pos, void* stream);

VVH_API int vvh_plan_run(vvh_plan plan, void* stream) { return plan_run(plan, 0, stream); }

VVH_API int vvh_plan_run_pos(vvh_plan plan, size_t pos, void* stream)
{
    if (pos > (size_t)INT64_MAX / 2) return fail(VVH_ERR_INVALID_ARG, "position %zu out of range", pos);
    return plan_run(plan, (int64_t)pos, stream);
}

static int plan_run(vvh_plan plan, int64_t pos, void* stream)
{
    REQUIRE_INIT();
    const Plan* p;
    {
        std::lock_guard<std::mutex> lock(g_pmu);
        auto it = g_plans.find(plan);
        if (it == g_plans.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown plan %llu", (unsigned long long)plan);
        p = &it->second;
    }
    if (p->dot) {
        // early launches load the activations with the weights (no LDS
        // staging) unless an input stage needs them in LDS
        const bool early = dot_early(p->total_blocks);
        const bool in_op = !p->args.empty() && p->args[0].xop != VVH_IN_NONE;
        const bool xl = p->x_in_lds && (in_op || !early);
        const int e = launch_dot_grouped(p->sargs.table, p->dev_block_prob, p->args.data(), (int)p->args.size(),
                                         p->total_blocks, p->max_m, xl, xl ? p->lds_bytes : (size_t)kDotRedBytes,
                                         p->out, early, p->dot_depth, pos, stream);
        return e == 0 ? VVH_OK : fail_hip((hipError_t)e, "grouped dot launch");
    }
    if (p->stream) {
        const int e = launch_stream(p->sargs, p->depth, p->max_m, p->out, ((int64_t)p->sargs.waves + 3) / 4, stream);
        return e == 0 ? VVH_OK : fail_hip((hipError_t)e, "streaming launch");
    }
    if (p->grouped) {
        const int e = launch_skinny_grouped(p->dev_table, (int)p->args.size(), p->total_blocks, p->out, stream);
        return e == 0 ? VVH_OK : fail_hip((hipError_t)e, "grouped launch");
    }
    for (const LinArgs& a : p->args) {
        const bool aligned = a.K % 16 == 0 && aligned16(a.w) && aligned16(a.inp);
        const int st = run_call(a, choose_kernel(a.M, a.N, a.K, p->act, aligned), p->act, p->out, stream);
        if (st != VVH_OK) return st;
    }
    return VVH_OK;
}

VVH_API int vvh_plan_set_input_op(vvh_plan plan, int in_op, const float* in_w, float in_eps)
{
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_pmu);
    auto it = g_plans.find(plan);
    if (it == g_plans.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown plan %llu", (unsigned long long)plan);
    Plan& p = it->second;
    if (!p.dot || !p.x_in_lds)
        return fail(VVH_ERR_UNSUPPORTED, "input stage needs a plan that runs as one k_dot_grouped launch "
                    "with its activations in LDS");
    for (const LinArgs& a : p.args) {
        const int st = input_op_ok(in_op, in_w, (std::size_t)a.M, (std::size_t)a.K, p.act);
        if (st != VVH_OK) return st;
    }
    for (LinArgs& a : p.args) {
        a.xop = in_op;
        a.xw = in_w;
        a.xeps = in_eps;
    }
    // the table is read by launches already queued: replace it once they are done
    (void)hipDeviceSynchronize();
    const hipError_t e = hipMemcpy(const_cast<LinArgs*>(p.sargs.table), p.args.data(), p.args.size() * sizeof(LinArgs),
                                   hipMemcpyHostToDevice);
    return e == hipSuccess ? VVH_OK : fail_hip(e, "plan table upload");
}

VVH_API int vvh_plan_set_rope(vvh_plan plan, size_t q_index, size_t k_index, size_t v_index, size_t head_dim,
                              float theta, void* k_cache, void* v_cache)
{
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_pmu);
    auto it = g_plans.find(plan);
    if (it == g_plans.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown plan %llu", (unsigned long long)plan);
    Plan& p = it->second;
    if (!p.dot) return fail(VVH_ERR_UNSUPPORTED, "RoPE epilogue needs a plan that runs as one k_dot_grouped launch");
    if (q_index == k_index || q_index == v_index || k_index == v_index)
        return fail(VVH_ERR_INVALID_ARG, "q, k and v must be different problems");
    if (!k_cache || !v_cache) return fail(VVH_ERR_INVALID_ARG, "k_cache and v_cache must be device pointers");
    if (head_dim < 16 || head_dim % 16 != 0 || head_dim > 4096)
        return fail(VVH_ERR_UNSUPPORTED, "RoPE epilogue needs head_dim a multiple of 16 (got %zu)", head_dim);
    if (!(theta > 0.0f) || !std::isfinite(theta)) return fail(VVH_ERR_INVALID_ARG, "theta must be positive");
    // the change is made on a copy of the plan's entries and becomes the
    // plan's only once the device table holds it, so a failed call (a
    // capture in progress, an allocation failure) leaves the plan as it was
    std::vector<LinArgs> next = p.args;
    LinArgs* q = nullptr;
    LinArgs* k = nullptr;
    LinArgs* v = nullptr;
    for (LinArgs& a : next) {
        if ((size_t)a.src == q_index) q = &a;
        if ((size_t)a.src == k_index) k = &a;
        if ((size_t)a.src == v_index) v = &a;
    }
    if (!q || !k || !v) return fail(VVH_ERR_INVALID_ARG, "q, k or v index names no (non-empty) problem of the plan");
    if (q->glu || k->glu || v->glu)
        return fail(VVH_ERR_INVALID_ARG, "a problem with the SiLU-gated epilogue cannot take RoPE");
    if (q->N > INT32_MAX || k->N > INT32_MAX)  // the epilogue maps tiles to row pairs in 32 bits
        return fail(VVH_ERR_UNSUPPORTED, "RoPE epilogue needs q and k rows below 2^31");
    if (q->N % (int64_t)head_dim != 0 || k->N % (int64_t)head_dim != 0 || k->N != v->N || k->M != v->M ||
        q->M != k->M)
        return fail(VVH_ERR_INVALID_ARG, "q rows (%lld), k and v rows (%lld, %lld) must be whole heads of %zu, with "
                    "k and v alike and one M", (long long)q->N, (long long)k->N, (long long)v->N, head_dim);
    // the table is read by launches already queued: replace it once they are done
    hipError_t fe = hipDeviceSynchronize();
    if (fe != hipSuccess) return fail_hip(fe, "plan RoPE epilogue: synchronize (no change made)");
    // the pair frequencies, worked out once on the device by the function
    // vvh_rope uses, and the cosine/sine table of position 0 (a longer one
    // comes from vvh_plan_set_rope_table)
    float* freq = nullptr;
    float* cs = nullptr;
    fe = hipMalloc(&freq, head_dim / 2 * sizeof(float));
    if (fe == hipSuccess) fe = hipMalloc(&cs, head_dim * sizeof(float));
    if (fe == hipSuccess) fe = (hipError_t)launch_rope_freq(freq, (int64_t)head_dim, theta, nullptr);
    if (fe == hipSuccess) fe = (hipError_t)launch_rope_table(cs, freq, 1, (int64_t)head_dim, nullptr);
    if (fe == hipSuccess) fe = hipDeviceSynchronize();
    if (fe != hipSuccess) {
        (void)hipGetLastError();
        if (freq) (void)hipFree(freq);
        if (cs) (void)hipFree(cs);
        return fail_hip(fe, "RoPE frequency table (no change made)");
    }
    q->rope = 1;
    k->rope = 2;
    v->rope = 3;
    for (LinArgs* a : {q, k, v}) {
        a->rope_d = (int32_t)head_dim;
        a->rope_theta = theta;
    }
    q->cache = nullptr;
    k->cache = k_cache;
    v->cache = v_cache;
    q->rope_freq = k->rope_freq = freq;
    q->rope_cs = k->rope_cs = cs;
    q->rope_cs_n = k->rope_cs_n = 1;
    const hipError_t e = hipMemcpy(const_cast<LinArgs*>(p.sargs.table), next.data(), next.size() * sizeof(LinArgs),
                                   hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        // the device table may hold part of the new entries: put the old ones back
        (void)hipGetLastError();
        (void)hipMemcpy(const_cast<LinArgs*>(p.sargs.table), p.args.data(), p.args.size() * sizeof(LinArgs),
                        hipMemcpyHostToDevice);
        (void)hipFree(freq);
        (void)hipFree(cs);
        return fail_hip(e, "plan table upload (no change made)");
    }
    if (p.rope_freq) p.rope_retired.push_back(p.rope_freq);
    if (p.rope_cs) p.rope_retired.push_back(p.rope_cs);
    p.rope_freq = freq;
    p.rope_cs = cs;
    p.rope_cs_n = 1;
    p.args = std::move(next);
    return VVH_OK;
}

VVH_API int vvh_plan_set_rope_table(vvh_plan plan, size_t positions)
{
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_pmu);
    auto it = g_plans.find(plan);
    if (it == g_plans.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown plan %llu", (unsigned long long)plan);
    Plan& p = it->second;
    if (!p.rope_freq) return fail(VVH_ERR_INVALID_ARG, "the plan has no RoPE epilogue (vvh_plan_set_rope first)");
    if (positions < 1 || positions > kRopeTableMaxPositions)
        return fail(VVH_ERR_INVALID_ARG, "RoPE table positions must be in [1, %lld] (got %zu)",
                    (long long)kRopeTableMaxPositions, positions);
    std::vector<LinArgs> next = p.args;
    int64_t d = 0;
    for (const LinArgs& a : next)
        if (a.rope == 1) d = a.rope_d;
    hipError_t fe = hipDeviceSynchronize();
    if (fe != hipSuccess) return fail_hip(fe, "plan RoPE table: synchronize (no change made)");
    float* cs = nullptr;
    fe = hipMalloc(&cs, positions * (size_t)d * sizeof(float));
    if (fe == hipSuccess) fe = (hipError_t)launch_rope_table(cs, p.rope_freq, (int64_t)positions, d, nullptr);
    if (fe == hipSuccess) fe = hipDeviceSynchronize();
    if (fe != hipSuccess) {
        (void)hipGetLastError();
        if (cs) (void)hipFree(cs);
        return fail_hip(fe, "RoPE cosine/sine table (no change made)");
    }
    for (LinArgs& a : next) {
        if (a.rope == 1 || a.rope == 2) {
            a.rope_cs = cs;
            a.rope_cs_n = (int64_t)positions;
        }
    }
    const hipError_t e = hipMemcpy(const_cast<LinArgs*>(p.sargs.table), next.data(), next.size() * sizeof(LinArgs),
                                   hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        (void)hipMemcpy(const_cast<LinArgs*>(p.sargs.table), p.args.data(), p.args.size() * sizeof(LinArgs),
                        hipMemcpyHostToDevice);
        (void)hipFree(cs);
        return fail_hip(e, "plan table upload (no change made)");
    }
    p.rope_retired.push_back(p.rope_cs);
    p.rope_cs = cs;
    p.rope_cs_n = (int64_t)positions;
    p.args = std::move(next);
    return VVH_OK;
}

VVH_API int vvh_plan_set_glu(vvh_plan plan, size_t index)
{
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_pmu);
    auto it = g_plans.find(plan);
    if (it == g_plans.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown plan %llu", (unsigned long long)plan);
    Plan& p = it->second;
    if (!p.dot)
        return fail(VVH_ERR_UNSUPPORTED, "SiLU-gated epilogue needs a plan that runs as one k_dot_grouped launch");
    LinArgs* g = nullptr;
    for (LinArgs& a : p.args)
        if ((size_t)a.src == index) g = &a;
    if (!g) return fail(VVH_ERR_INVALID_ARG, "index %zu names no (non-empty) problem of the plan", index);
    if (g->N % 16 != 0)
        return fail(VVH_ERR_UNSUPPORTED, "SiLU-gated epilogue needs N = 2 * inter with inter %% 8 == 0 (N %lld)",
                    (long long)g->N);
    if (g->res) return fail(VVH_ERR_INVALID_ARG, "SiLU-gated epilogue takes no residual");
    if (g->rope) return fail(VVH_ERR_INVALID_ARG, "a problem with a RoPE epilogue cannot be SiLU-gated");
    // the table is read by launches already queued: replace it once they
    // are done; the plan's entries change only once the upload succeeded
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail_hip(e, "plan SiLU-gated epilogue: synchronize (no change made)");
    std::vector<LinArgs> next = p.args;
    next[(size_t)(g - p.args.data())].glu = 1;
    e = hipMemcpy(const_cast<LinArgs*>(p.sargs.table), next.data(), next.size() * sizeof(LinArgs),
                  hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        (void)hipMemcpy(const_cast<LinArgs*>(p.sargs.table), p.args.data(), p.args.size() * sizeof(LinArgs),
                        hipMemcpyHostToDevice);
        return fail_hip(e, "plan table upload (no change made)");
    }
    p.args = std::move(next);
    return VVH_OK;
}

VVH_API int vvh_plan_destroy(vvh_plan plan)
{
    std::lock_guard<std::mutex> lock(g_pmu);
    auto it = g_plans.find(plan);
    if (it == g_plans.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown plan %llu", (unsigned long long)plan);
    if (it->second.dev_table) (void)hipFree(it->second.dev_table);
    if (it->second.dev_stream) (void)hipFree(it->second.dev_stream);
    if (it->second.rope_freq) (void)hipFree(it->second.rope_freq);
    if (it->second.rope_cs) (void)hipFree(it->second.rope_cs);
    for (float* t : it->second.rope_retired) (void)hipFree(t);
    g_plans.erase(it);
    return VVH_OK;
}

VVH_API int vvh_plan_launches(vvh_plan plan, int* launches)
{
    if (!launches) return fail(VVH_ERR_INVALID_ARG, "launches is null");
    std::lock_guard<std::mutex> lock(g_pmu);
    auto it = g_plans.find(plan);
    if (it == g_plans.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown plan %llu", (unsigned long long)plan);
    *launches = (it->second.grouped || it->second.stream || it->second.dot) ? 1 : (int)it->second.args.size();
    return VVH_OK;
}

VVH_API int vvh_plan_kernel(vvh_plan plan, int* kernel)
{
    if (!kernel) return fail(VVH_ERR_INVALID_ARG, "kernel is null");
    std::lock_guard<std::mutex> lock(g_pmu);
    auto it = g_plans.find(plan);
    if (it == g_plans.end()) return fail(VVH_ERR_UNKNOWN_HANDLE, "unknown plan %llu", (unsigned long long)plan);
    *kernel = it->second.dot ? K_DOT : it->second.stream ? K_STREAM : it->second.grouped ? K_SKINNY : K_AUTO;
    return VVH_OK;
}

// ---- quantizer, conversion, synthetic data ---------------------------------------------------
VVH_API int vvh_quantize_per_channel(const float* dev_weight, size_t N, size_t K, int8_t* dev_codes,
                                     float* dev_scales, void* stream)
{
    uint64_t nk;
    if (!mul_ok(N, K, &nk)) return fail(VVH_ERR_INVALID_ARG, "size overflow");
    if (N == 0) return VVH_OK;
    if (!dev_scales || (K > 0 && (!dev_weight || !dev_codes)))
        return fail(VVH_ERR_INVALID_ARG, "null pointer");
    REQUIRE_INIT();
    const int e = launch_quantize(dev_weight, VVH_F32, (int64_t)N, (int64_t)K, dev_codes, dev_scales, stream);
    return e == 0 ? VVH_OK : fail_hip((hipError_t)e, "quantize launch");
}

VVH_API int vvh_convert(void* dst, int dst_dtype, const void* src, int src_dtype, size_t n, void* stream)
{
    if (!valid_dtype(dst_dtype) || !valid_dtype(src_dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (n == 0) return VVH_OK;
    if (!dst || !src) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (n > (uint64_t(1) << 61)) return fail(VVH_ERR_INVALID_ARG, "size overflow");
    REQUIRE_INIT();
    const int e = launch_convert(dst, dst_dtype, src, src_dtype, (int64_t)n, stream);
    return e == 0 ? VVH_OK : fail_hip((hipError_t)e, "convert launch");
}

VVH_API int vvh_fill_normal(void* dst, int dtype, size_t n, uint64_t seed, float mean, float std, void* stream)
{
    if (!valid_dtype(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (n == 0) return VVH_OK;
    if (!dst) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (n > (uint64_t(1) << 61)) return fail(VVH_ERR_INVALID_ARG, "size overflow");
    REQUIRE_INIT();
    const int e = launch_fill_normal(dst, dtype, (int64_t)n, seed, mean, std, stream);
    return e == 0 ? VVH_OK : fail_hip((hipError_t)e, "fill launch");
}

// ---- dispatch introspection --------------------------------------------------------------------
VVH_API int vvh_linear_q8_choice(size_t M, size_t N, size_t K, int act_dtype, int out_dtype)
{
    if (!valid_dtype(act_dtype) || !valid_dtype(out_dtype)) return -fail(VVH_ERR_INVALID_ARG, "bad dtype");
    return choose_kernel(M, N, K, act_dtype, K % 16 == 0);
}

VVH_API int vvh_gemm_variant(size_t M, size_t N, size_t K, int* tile_n, int* splits)
{
    if (M == 0 || N == 0) return -fail(VVH_ERR_INVALID_ARG, "empty problem");
    int tn = kGemmBN, s = 1, v = 1;
    if (K % kGemmBK == 0) {
        const int64_t stages = (int64_t)K / kGemmBK;
        int split_layout = 4;
        s = gemm_splits((int64_t)M, (int64_t)N, stages, &split_layout);
        if (s > 1) {  // as the dispatch: no empty split
            const int64_t kst = (stages + s - 1) / s;
            s = (int)((stages + kst - 1) / kst);
        }
        const int layout = gemm3_layout((int64_t)M, (int64_t)N, s, split_layout);
        v = gemm3_tile_m(layout) == 64 ? 4 : 3;
        tn = gemm3_tile_n(layout);
    }
    if (tile_n) *tile_n = tn;
    if (splits) *splits = s;
    return v;
}

VVH_API int vvh_set_kernel_override(int kernel)
{
    if (kernel < K_AUTO || kernel > K_DOT) return fail(VVH_ERR_INVALID_ARG, "bad kernel %d", kernel);
    g_override.store(kernel);
    return VVH_OK;
}


// ---- the other operators of a decode step --------------------------------------------------
namespace {
struct ArrayMirror {
    void* dev = nullptr;
    std::size_t n = 0;
};
std::mutex g_amu;
std::unordered_map<const float*, ArrayMirror> g_arr[2];  // [0]: fp32 copies, [1]: fp16 copies

inline int act_ok(int dtype) { return dtype == VVH_F32 || dtype == VVH_F16; }
inline int ret_launch(int e, const char* what) { return e == 0 ? VVH_OK : fail_hip((hipError_t)e, what); }

VVH_API int vvh_kv_append(void* k_dst, void* v_dst, const void* k_src, const void* v_src, size_t bytes, void* stream)
{
    if (bytes == 0) return VVH_OK;
    if (!k_dst || !v_dst || !k_src || !v_src) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (bytes > (size_t)INT64_MAX / 2) return fail(VVH_ERR_INVALID_ARG, "size overflow");
    REQUIRE_INIT();
    return ret_launch(launch_copy2(k_dst, k_src, v_dst, v_src, (int64_t)bytes, stream), "kv append launch");
}
}  // namespace

VVH_API int vvh_eltwise(int op, void* out, const void* x, const void* y, size_t n, int dtype, void* stream)
{
    if (op < VVH_OP_ADD || op > VVH_OP_SILU_MUL || !act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad op or dtype");
    if (n == 0) return VVH_OK;
    if (!out || !x || (op != VVH_OP_SILU && !y)) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    REQUIRE_INIT();
    return ret_launch(launch_eltwise(op, out, x, y, (int64_t)n, dtype, stream), "eltwise launch");
}

VVH_API int vvh_rms_norm(void* out, const void* x, const float* dev_weight, size_t rows, size_t n, float eps,
                         int dtype, void* stream)
{
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (rows == 0 || n == 0) return VVH_OK;
    if (!out || !x || !dev_weight) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (rows > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "too many rows");
    REQUIRE_INIT();
    return ret_launch(launch_rms_norm(out, x, dev_weight, (int64_t)rows, (int64_t)n, eps, dtype, stream), "rms_norm launch");
}

VVH_API int vvh_softmax(void* out, const void* x, size_t rows, size_t n, int dtype, void* stream)
{
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (rows == 0 || n == 0) return VVH_OK;
    if (!out || !x) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (rows > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "too many rows");
    REQUIRE_INIT();
    return ret_launch(launch_softmax(out, x, (int64_t)rows, (int64_t)n, dtype, stream), "softmax launch");
}

VVH_API int vvh_rope(void* q, void* k, size_t seq_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
                     size_t pos, float theta, int dtype, void* stream)
{
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (head_dim % 2 != 0) return fail(VVH_ERR_INVALID_ARG, "odd head_dim %zu", head_dim);
    if (seq_len == 0 || head_dim == 0 || (num_heads == 0 && num_kv_heads == 0)) return VVH_OK;
    if ((num_heads && !q) || (num_kv_heads && !k)) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    REQUIRE_INIT();
    return ret_launch(launch_rope(q, k, (int64_t)seq_len, (int64_t)num_heads, (int64_t)num_kv_heads, (int64_t)head_dim,
                                  (int64_t)pos, theta, dtype, stream),
                      "rope launch");
}

VVH_API int vvh_rope_append(void* q, void* k, const void* v, void* k_cache, void* v_cache, size_t seq_len,
                            size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t pos, float theta, int dtype,
                            void* stream)
{
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (head_dim % 2 != 0) return fail(VVH_ERR_INVALID_ARG, "odd head_dim %zu", head_dim);
    if (seq_len == 0 || head_dim == 0 || (num_heads == 0 && num_kv_heads == 0)) return VVH_OK;
    if ((num_heads && !q) || (num_kv_heads && (!k || !v || !k_cache || !v_cache)))
        return fail(VVH_ERR_INVALID_ARG, "null pointer");
    REQUIRE_INIT();
    return ret_launch(launch_rope_append(q, k, v, k_cache, v_cache, (int64_t)seq_len, (int64_t)num_heads,
                                         (int64_t)num_kv_heads, (int64_t)head_dim, (int64_t)pos, theta, dtype, stream),
                      "rope append launch");
}

VVH_API int vvh_embedding(void* out, const float* dev_table, size_t token_id, size_t hidden, size_t vocab, int dtype,
                          void* stream)
{
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (token_id >= vocab) return fail(VVH_ERR_INVALID_ARG, "token %zu out of range (vocab %zu)", token_id, vocab);
    if (hidden == 0) return VVH_OK;
    if (!out || !dev_table) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    REQUIRE_INIT();
    return ret_launch(launch_embedding(out, dev_table, (int64_t)token_id, (int64_t)hidden, dtype, stream),
                      "embedding launch");
}

VVH_API int vvh_attention(void* out, const void* q, const void* k, const void* v, size_t n_q, size_t len0,
                          size_t num_heads, size_t num_kv_heads, size_t head_dim, float scale, int dtype, void* stream)
{
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (n_q == 0 || num_heads == 0) return VVH_OK;
    if (!out || !q || !k || !v) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0)
        return fail(VVH_ERR_INVALID_ARG, "num_heads %zu not a multiple of num_kv_heads %zu", num_heads, num_kv_heads);
    if (head_dim == 0 || head_dim > 256) return fail(VVH_ERR_INVALID_ARG, "head_dim %zu outside 1..256", head_dim);
    if (len0 == 0) return fail(VVH_ERR_INVALID_ARG, "a query attends to at least one position");
    if (num_heads > 65535 || n_q > 65535) return fail(VVH_ERR_UNSUPPORTED, "grid too large");
    const bool decode = n_q == 1 && attention_decode_ok(k, v, (int64_t)len0, (int64_t)num_heads,
                                                        (int64_t)num_kv_heads, (int64_t)head_dim);
    if (!decode && len0 + n_q - 1 > (size_t)attention_max_len())
        return fail(VVH_ERR_UNSUPPORTED, "attention span %zu > %lld", len0 + n_q - 1, (long long)attention_max_len());
    REQUIRE_INIT();
    if (decode) {
        const AttnDecodePlan p = attention_decode_plan(q, (int64_t)len0, (int64_t)num_heads, (int64_t)num_kv_heads,
                                                       (int64_t)head_dim, dtype);
        float* ws = nullptr;
        unsigned* cnt = nullptr;
        const int64_t wsf = attention_decode_ws_floats(p, (int64_t)num_heads, (int64_t)head_dim);
        if (wsf > 0) {
            const int st = workspace_for(stream, (std::size_t)wsf * 4, &ws);
            if (st != VVH_OK) return st;
        }
        if (attention_decode_counted(p)) {
            const int st = counters_for(stream, &cnt);
            if (st != VVH_OK) return st;
        }
        return ret_launch(launch_attention_decode(p, out, q, k, v, (int64_t)len0, (int64_t)num_heads,
                                                  (int64_t)num_kv_heads, (int64_t)head_dim, scale, ws, cnt, dtype,
                                                  stream),
                          "attention launch");
    }
    return ret_launch(launch_attention(out, q, k, v, (int64_t)n_q, (int64_t)len0, (int64_t)num_heads,
                                       (int64_t)num_kv_heads, (int64_t)head_dim, scale, dtype, stream),
                      "attention launch");
}

VVH_API int vvh_attention_parts(float* parts, size_t parts_floats, size_t* nparts, const void* q, const void* k,
                                const void* v, size_t len0, size_t num_heads, size_t num_kv_heads,
                                size_t head_dim, float scale, int dtype, void* stream)
{
    if (!nparts) return fail(VVH_ERR_INVALID_ARG, "nparts is null");
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (!parts || !q || !k || !v) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (num_heads == 0 || num_kv_heads == 0 || num_heads % num_kv_heads != 0)
        return fail(VVH_ERR_INVALID_ARG, "num_heads %zu not a multiple of num_kv_heads %zu", num_heads, num_kv_heads);
    if (len0 == 0) return fail(VVH_ERR_INVALID_ARG, "a query attends to at least one position");
    if (dtype != VVH_F16 || (head_dim != 64 && head_dim != 128) || num_heads > 65535 ||
        !attention_decode_ok(k, v, (int64_t)len0, (int64_t)num_heads, (int64_t)num_kv_heads, (int64_t)head_dim) ||
        !aligned16(parts))
        return fail(VVH_ERR_UNSUPPORTED, "attention parts need fp16, head_dim 64 or 128, num_heads / num_kv_heads "
                    "<= 16 and 16-byte aligned q, k, v and parts");
    const AttnDecodePlan p = attention_decode_plan(q, (int64_t)len0, (int64_t)num_heads, (int64_t)num_kv_heads,
                                                   (int64_t)head_dim, dtype);
    if (!p.mfma || p.nb != 1)
        return fail(VVH_ERR_UNSUPPORTED, "a span of %zu positions is not one block per kv head (at most 512)", len0);
    const std::size_t need = (std::size_t)p.waves * num_heads * (head_dim + 4);
    if (parts_floats < need)
        return fail(VVH_ERR_INVALID_ARG, "parts holds %zu floats, %zu needed", parts_floats, need);
    REQUIRE_INIT();
    const int st = ret_launch(launch_attention_parts(parts, q, k, v, (int64_t)len0, (int64_t)num_heads,
                                                     (int64_t)num_kv_heads, (int64_t)head_dim, scale, p.waves, stream),
                              "attention parts launch");
    if (st == VVH_OK) *nparts = (std::size_t)p.waves;
    return st;
}

VVH_API int vvh_dense(void* out, const void* x, const void* dev_weight, int wdtype, const float* dev_bias,
                      const void* residual, size_t M, size_t N, size_t K, int dtype, void* stream)
{
    if (!act_ok(dtype) || !act_ok(wdtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    uint64_t t;
    if (!mul_ok(M, N, &t) || !mul_ok(N, K, &t) || !mul_ok(M, K, &t)) return fail(VVH_ERR_INVALID_ARG, "size overflow");
    if (M == 0 || N == 0) return VVH_OK;
    if (!out || (K > 0 && (!x || !dev_weight))) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if ((N + 3) / 4 > INT32_MAX) return fail(VVH_ERR_UNSUPPORTED, "N too large");
    REQUIRE_INIT();
    return ret_launch(launch_dense(out, x, dev_weight, wdtype, dev_bias, residual, (int64_t)M, (int64_t)N, (int64_t)K,
                                   dtype, stream),
                      "dense launch");
}

VVH_API int vvh_matmul(void* out, const void* A, const float* dev_B, size_t M, size_t N, size_t K, int dtype,
                       void* stream)
{
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    uint64_t t;
    if (!mul_ok(M, N, &t) || !mul_ok(K, N, &t) || !mul_ok(M, K, &t)) return fail(VVH_ERR_INVALID_ARG, "size overflow");
    if (M == 0 || N == 0) return VVH_OK;
    if (!out || (K > 0 && (!A || !dev_B))) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    REQUIRE_INIT();
    return ret_launch(launch_matmul(out, A, dev_B, (int64_t)M, (int64_t)N, (int64_t)K, dtype, stream), "matmul launch");
}

VVH_API int vvh_argmax(const float* logits, size_t n, int32_t* dev_index, void* stream)
{
    if (!logits || !dev_index) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (n == 0 || n > INT32_MAX) return fail(VVH_ERR_INVALID_ARG, "bad length %zu", n);
    REQUIRE_INIT();
    float* ws = nullptr;
    const int64_t wsb = argmax_ws_bytes((int64_t)n);
    if (wsb > 0) {
        const int st = workspace_for(stream, (std::size_t)wsb, &ws);
        if (st != VVH_OK) return st;
    }
    return ret_launch(launch_argmax(logits, (int64_t)n, dev_index, ws, stream), "argmax launch");
}

VVH_API int vvh_sample(const void* logits, int dtype, size_t n, float temperature, float top_p, uint64_t seed,
                       int32_t step, int32_t* dev_index, void* stream)
{
    (void)top_p;  // accepted and ignored, as cuda_sample does (src/backend/cuda_kernels.cu:1325)
    if (!act_ok(dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    if (!logits || !dev_index) return fail(VVH_ERR_INVALID_ARG, "null pointer");
    if (n == 0 || n > INT32_MAX) return fail(VVH_ERR_INVALID_ARG, "bad length %zu", n);
    if (!(temperature >= 0.0f) || temperature == INFINITY)
        return fail(VVH_ERR_INVALID_ARG, "temperature %g is not a finite value >= 0", (double)temperature);
    REQUIRE_INIT();
    float* ws = nullptr;
    const int64_t wsb = argmax_ws_bytes((int64_t)n);
    if (wsb > 0) {
        const int st = workspace_for(stream, (std::size_t)wsb, &ws);
        if (st != VVH_OK) return st;
    }
    return ret_launch(launch_sample(logits, dtype, (int64_t)n, temperature, seed, step, dev_index, ws, stream),
                      "sample launch");
}

VVH_API int vvh_mirror_f32(const float* host, size_t n, int as_dtype, const void** dev)
{
    if (!dev) return fail(VVH_ERR_INVALID_ARG, "dev is null");
    *dev = nullptr;
    if (!host || n == 0) return fail(VVH_ERR_INVALID_ARG, "empty host array");
    if (!act_ok(as_dtype)) return fail(VVH_ERR_INVALID_ARG, "bad dtype");
    uint64_t bytes;
    if (!mul_ok(n, 4, &bytes)) return fail(VVH_ERR_INVALID_ARG, "size overflow");
    REQUIRE_INIT();
    std::lock_guard<std::mutex> lock(g_amu);
    auto& map = g_arr[as_dtype == VVH_F16 ? 1 : 0];
    auto it = map.find(host);
    if (it != map.end()) {
        if (it->second.n == n) {
            *dev = it->second.dev;
            return VVH_OK;
        }
        (void)hipDeviceSynchronize();  // the old copy may still be read by queued work
        (void)hipFree(it->second.dev);
        map.erase(it);
    }
    void* d = nullptr;
    hipError_t e = hipMalloc(&d, as_dtype == VVH_F16 ? n * 2 : n * 4);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail_hip(e, "mirror hipMalloc");
    }
    if (as_dtype == VVH_F32) {
        e = hipMemcpy(d, host, n * 4, hipMemcpyHostToDevice);
    } else {  // upload fp32, convert on the device
        void* tmp = nullptr;
        e = hipMalloc(&tmp, n * 4);
        if (e == hipSuccess) e = hipMemcpy(tmp, host, n * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) {
            const int k = launch_convert(d, VVH_F16, tmp, VVH_F32, (int64_t)n, nullptr);
            e = k ? (hipError_t)k : hipDeviceSynchronize();
        }
        if (tmp) (void)hipFree(tmp);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(d);
        return fail_hip(e, "mirror upload");
    }
    map[host] = ArrayMirror{d, n};
    *dev = d;
    return VVH_OK;
}

VVH_API int vvh_mirror_release(const float* host)
{
    std::lock_guard<std::mutex> lock(g_amu);
    bool found = false;
    for (auto& map : g_arr) {
        auto it = map.find(host);
        if (it == map.end()) continue;
        if (!found) (void)hipDeviceSynchronize();
        (void)hipFree(it->second.dev);
        map.erase(it);
        found = true;
    }
    return found ? VVH_OK : fail(VVH_ERR_UNKNOWN_HANDLE, "no mirror of %p", (const void*)host);
}

}  // extern "C"
