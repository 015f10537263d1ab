// Internal declarations shared by the runtime and the kernels of
// libvvllm_hip.so.  Nothing here is part of the public C ABI
// (include/vvllm_hip.h).
#pragma once

#include <cstddef>
#include <cstdint>

#include "vvllm_hip.h"

namespace vvh {

// One linear_q8 problem as the kernels see it.  All pointers are device
// pointers; `inp`/`out`/`res` carry the element types the launcher was
// instantiated for.  Sizes are 64-bit: a single weight may exceed 2^31 codes
// on a 288 GB device.
struct LinArgs {
    void* out;
    const void* inp;
    const void* res;          // may be null; may alias out
    const int8_t* w;          // [N, K] codes
    const float* scales;      // [N]
    const float* bias;        // [N] or null
    int64_t M, N, K;
    int32_t ksplit;           // decode kernels: waves cooperating on one 16-row tile (1, 2, 4)
    int32_t block_begin;      // grouped launch: first block of this problem
    int64_t tile_begin;       // streaming plan: first global 16-row tile of this problem
    // GEMM split-K: nsplit blocks share each output tile, each running
    // kstages 64-wide k stages; their raw fp32 sums go to ws[split][M][N]
    // and k_splitk_reduce applies the epilogue.  nsplit <= 1: no split.
    float* ws;
    int32_t nsplit;
    int32_t kstages;
    // GEMM tile numbering: 0 = row blocks fastest (consecutive tiles share
    // their codes), 1 = column blocks fastest (consecutive tiles share their
    // activation rows); each XCD runs a contiguous range of tiles
    int32_t norder;
    // k_dot input stage (activations staged in LDS only): xop 0 = inp as is,
    // 1 = RMSNorm of each row of inp with weights xw and epsilon xeps (the
    // arithmetic of k_rms_norm), 2 = silu(gate) * up of rows [gate | up] of
    // 2K values (the arithmetic of k_eltwise's SiLU-mul),
    // 3 = the merge of decode-attention parts (one activation row): inp holds
    // xparts blocks of K / xhd part rows of xhd + 4 floats [O, m, l, -, -]
    // (k_attention_parts), element h xhd + d of the row is the merge of the
    // parts of head h.
    const float* xw;
    float xeps;
    int32_t xop;
    int32_t xparts;
    int32_t xhd;
    // q/k/v plan epilogue with RoPE and the KV-cache append (k_dot plans,
    // vvh_plan_set_rope): rope 0 = plain store; 1 = q rows, rotated; 2 = k
    // rows, rotated and also written to row pos + m of `cache`; 3 = v rows,
    // also written to row pos + m of `cache`.  For 1 and 2 a tile of head h
    // holds the row pairs (h*rope_d + 8s + r, + rope_d/2), r < 8, so each lane
    // owns the two halves of its rotation.
    int32_t rope;
    int32_t rope_d;
    float rope_theta;
    void* cache;
    const float* rope_freq;  // q and k rows: rope_freq(i, rope_d, rope_theta) for i < rope_d / 2
    // q and k rows: rope_cs of pair i at position p in rope_cs[2 (p rope_d / 2
    // + i)] (cosine) and the float after it (sine) for p < rope_cs_n
    // (rope_cs_n >= 1); positions past the table work them out from rope_freq
    const float* rope_cs;
    int64_t rope_cs_n;
    int32_t src;  // plans: index of the problem in the caller's list
    // plans: 1 = SiLU-gated epilogue: the N rows are [gate | up] of N / 2
    // each and out gets M rows of N / 2 values silu(gate) * up
    int32_t glu;
    // fp32 activations on the GEMM: inp holds M rows of 2 * bk fp16 values
    // (K = 2 * bk), the high and low fp16 parts of each fp32 activation
    // scaled by a power of two, and xrs[m] = that row's inverse scale; the
    // codes have rows of bk (0: K).
    int64_t bk;
    const float* xrs;
};

// k_dot_grouped: a plan of at most kDotInline problems passes its table in
// the kernel arguments, so a block finds its problem without a memory load.
constexpr int kDotInline = 4;
struct DotGroup {
    LinArgs p[kDotInline];
};

// Persistent streaming decode launch (k_stream).  Work is a sequence of
// 16-row tiles (one tile = 16 output channels x the full K).  Every wave
// walks its own tiles, keeping a fixed number of weight loads in flight
// across tile boundaries.
//   mode kStreamRange: one problem (`one`); wave w takes the contiguous
//                      tiles [T*w/W, T*(w+1)/W).
//   mode kStreamList:  a plan; wave w takes the global tiles
//                      list[list_off[w] .. list_off[w+1]), and
//                      tile_prob[g] is the problem of global tile g.
struct StreamArgs {
    LinArgs one;
    const LinArgs* table;
    const int32_t* tile_prob;
    const int32_t* list;
    const int32_t* list_off;
    int64_t total_tiles;
    int32_t waves;
    int32_t mode;
};
constexpr int kStreamRange = 0;
constexpr int kStreamList = 1;

// Kernel families (values match vvh_kernel).
enum Kernel : int {
    K_AUTO = VVH_KERNEL_AUTO,
    K_GENERIC = VVH_KERNEL_GENERIC,
    K_GEMV_F32 = VVH_KERNEL_GEMV_F32,
    K_SKINNY = VVH_KERNEL_SKINNY,
    K_GEMM = VVH_KERNEL_GEMM,
    K_STREAM = VVH_KERNEL_STREAM,
    K_DOT = VVH_KERNEL_DOT,
};

// Largest M served by the decode kernels.
constexpr int64_t kSkinnyMaxM = 16;   // one 16-row MFMA operand (grouped launches, k_stream)
constexpr int64_t kSkinnyMgMaxM = 64;  // single k_skinny calls: up to 4 groups of 16 rows
constexpr int64_t kGemvF32MaxM = 8;   // rows of fp32 activations per pass

// Rows of output channels handled by one wave of the decode kernels.
constexpr int kDecodeTileN = 16;

// Number of blocks a decode-kernel launch needs for one problem.
inline int64_t decode_blocks(const LinArgs& a)
{
    const int64_t tiles = (a.N + kDecodeTileN - 1) / kDecodeTileN;
    const int64_t tiles_per_block = 4 / a.ksplit;
    return (tiles + tiles_per_block - 1) / tiles_per_block;
}

// k_dot (M <= 16): 16-row tiles, 128-wide k steps, ksplit waves per tile.
constexpr int64_t kDotMaxM = 16;
constexpr int kStageMaxM = 4;  // rows of a decode linear with an input stage
// longest cosine/sine table of a plan's RoPE epilogue (vvh_plan_set_rope_table)
constexpr int64_t kRopeTableMaxPositions = (int64_t)1 << 20;
// attention merge stage: at most kAttnMaxParts parts, K <= kAttnMergeMaxK (4 per thread)
constexpr int kAttnMaxParts = 8;
constexpr int kAttnMergeMaxK = 1024;
constexpr int kDotStep = 128;               // k codes per row per step
constexpr int64_t kDotLdsMax = 80 * 1024;   // dynamic LDS of one block at most
constexpr int64_t kDotRedBytes = 4 * kDotMaxM * 16 * 4;
// k_dot with 3 to 16 activation rows (MT = 4, 8 or 16) takes its dot products on MFMA:
// each wave passes its step's 16 x 128 code tile through LDS (rows of
// kDotWtPitch bytes) to gather the MFMA operand fragments
constexpr int kDotWtPitch = 144;
constexpr int64_t kDotWtBytes = 4 * 16 * kDotWtPitch;
// ... and, when its activations are not staged in LDS, loads them in whole
// 128-byte lines (8 rows per instruction) and passes each step's rows of
// 128 values through a per-wave LDS tile (rows of kDotXtPitch bytes) too
constexpr int kDotXtPitch = 272;
constexpr int64_t kDotXtBytes = 4 * 16 * kDotXtPitch;
// k_dot's activation source: staged in LDS, loaded with the weights as MFMA
// operands (or per row for M <= 2), or loaded with the weights in whole lines
// and regathered through the wave's LDS tile (MFMA path only)
constexpr int kXDirect = 0, kXLds = 1, kXTile = 2;
// The tile pays where a launch's tiles re-read many activation bytes (each
// 16-row tile reads all M rows): from about 5 MB (graph replay, A/B of both
// sources: 1.5B gate 8960 x 1536 at M = 16 9.6 -> 8.4 us, at M = 4 7.0 ->
// 6.5; 0.5B down 896 x 4864 at M = 16 8.5 -> 7.9; 0.5B q at M = 4 3.16 ->
// 3.40 and down at M = 4 6.2 -> 6.5 below the threshold).
// Waves with long k ranges pay the regathering once per step in series, so
// it needs at most kDotXTileSteps steps per wave (1.5B down 1536 x 8960 at
// M = 4, 18 steps per wave: 8.95 -> 9.47 us with it; 0.5B down at M = 16,
// 10 steps: 8.5 -> 7.9 us).
constexpr int64_t kDotXTileBytes = 5ll << 20;
constexpr int64_t kDotXTileSteps = 12;
inline int64_t dot_x_reread_bytes(int64_t M, int64_t N, int64_t K)
{
    return ((N + kDecodeTileN - 1) / kDecodeTileN) * M * K * 2;
}
inline int64_t dot_wave_steps(int64_t K, int32_t ksplit)
{
    const int64_t steps = (K + kDotStep - 1) / kDotStep;
    return (steps + ksplit - 1) / (ksplit > 0 ? ksplit : 1);
}
// k_dot's k split 8 (blocks of 8 waves, one tile each) for plain calls of
// 9-16 rows (the MFMA path, activations loaded with the weights) over at
// most one block per CU whose waves would have exactly 3 k steps each at
// k split 4 (K of 1025-1536): graph replay, 1.5B q/o 1536 x 1536 at M = 16
// 4.64 -> 4.44 us, k/v 256 x 1536 4.49 -> 4.30.  On longer rows the second
// wave per SIMD costs more than the shorter chain saves (0.5B down 896 x
// 4864 at M = 8 / 16: 6.42 / 7.56 -> 8.09 / 9.01 us; 1.5B down at M = 8
// 9.46 -> 9.75), on rows of 2 steps per wave at split 4 it loses too
// (0.5B q/o 896 x 896 at M = 16 3.61 -> 4.45 us, 1024 x 1024 3.61 -> 4.68),
// and at 8 rows it gains nothing (q/o 4.08 -> 4.06).
inline bool dot_split8(int64_t M, int64_t tiles, int64_t K, int64_t cus)
{
    return M > 8 && M <= kDotMaxM && tiles <= cus && dot_wave_steps(K, 4) == 3;
}
// The activation tile's rule, for a launch of max_m rows whose problems
// re-read `reread` activation bytes over their tiles and give a wave at most
// `wave_steps` k steps (launch_dot, launch_dot_grouped and the dispatcher).
inline bool dot_takes_x_tile(int64_t max_m, bool early, bool x_in_lds, int64_t reread, int64_t wave_steps)
{
    return max_m > 2 && early && !x_in_lds && reread >= kDotXTileBytes && wave_steps <= kDotXTileSteps;
}
// k_dot takes N, M and K as 32-bit kernel arguments and 32-bit k offsets
inline bool dot_fits(int64_t N, int64_t K)
{
    return N <= INT32_MAX && K <= INT32_MAX - kDotStep;
}
inline int64_t dot_blocks(const LinArgs& a)
{
    const int64_t tiles = (a.N + kDecodeTileN - 1) / kDecodeTileN;
    const int64_t tiles_per_block = (a.ksplit > 4 ? 8 : 4) / a.ksplit;  // blocks of 4 waves, of 8 at k split 8
    return (tiles + tiles_per_block - 1) / tiles_per_block;
}
// Activations are staged in LDS when M rows of K + 8 halves fit beside the
// reduction scratch; the launcher and the kernel both use this rule.
inline __host__ __device__ bool dot_x_in_lds(int64_t M, int64_t K)
{
    return kDotRedBytes + M * (K + 8) * 2 <= kDotLdsMax;
}
inline __host__ __device__ int64_t dot_lds_bytes(int64_t M, int64_t K)
{
    return kDotRedBytes + (dot_x_in_lds(M, K) ? M * (K + 8) * 2 : 0);
}
// k_dot first stages (requested ahead of the weight ring, a template
// parameter of the kernel): none, RMSNorm (xop 1, M <= 4, K <= 2048), the
// attention merge (xop 3), plain activations (xop 0, M = 1)
constexpr int kFirstNone = 0;
constexpr int kFirstRms = 1;   // rows of K <= 1024 (2 chunks of 8 per lane)
constexpr int kFirstRms4 = 2;  // rows of K <= 2048 (4 chunks per lane)
constexpr int kFirstAttn = 3;
// k_dot_grouped epilogue kinds (a template parameter): every epilogue behind
// run-time tests, or only the plain store, the SiLU-gated or the RoPE one
constexpr int kEpiAny = 0;
constexpr int kEpiPlain = 1;
constexpr int kEpiGlu = 2;
constexpr int kEpiRope = 3;
inline int dot_first_rms(int64_t M, int64_t K)
{
    if (M > 4 || K % 16 != 0 || !dot_x_in_lds(M, K)) return kFirstNone;
    return K <= 1024 ? kFirstRms : K <= 2048 ? kFirstRms4 : kFirstNone;
}
// plain activations of one to four rows staged in LDS, requested ahead of
// the ring in 1, 3 or 5 rounds of 256 chunks of 8 halves (M K <= 2048,
// 6144, 10240), for launches of at most kDotXFirstMaxBlocks blocks (3-4
// rows: K >= 1024 only; graph replay, 1.5B q/o at M = 3 / 4 3.82 / 3.90 ->
// 3.67, k/v 3.66 / 3.70 -> 3.48, gate at M = 3 6.77 -> 6.15 us, while the
// 0.5B q/k/v/o/gate (K = 896, two k steps per wave) lost 0.1-0.2 us; 5-16
// rows in up to 12 rounds measured slower: 1.5B q/o at M = 12 / 16 4.35 /
// 4.65 -> 4.95 / 5.30 us, 0.5B down at M = 5 6.2 -> 7.0).
// Graph-replayed at M = 1 against the activations in the ring: 1.5B gate
// 8960 x 1536 (560 blocks) 5.57 -> 5.28 us, q/o 3.05 -> 2.98, down 7.1 ->
// 6.98, the 0.5B shapes unchanged, the LM head (2374 blocks, each with a
// barrier more) 23.1 -> 23.4.
constexpr int kFirstX1 = 4;
constexpr int kFirstX3 = 5;
constexpr int kFirstX5 = 6;
constexpr int64_t kDotXFirstMaxBlocks = 1024;
inline int dot_first_x(int64_t M, int64_t K, int64_t blocks)
{
    if (M < 1 || M > 4 || (M > 2 && K < 1024) || blocks > kDotXFirstMaxBlocks) return kFirstNone;
    const int64_t rounds = (M * K / 8 + 255) / 256;
    return rounds <= 1 ? kFirstX1 : rounds <= 3 ? kFirstX3 : rounds <= 5 ? kFirstX5 : kFirstNone;
}

// GEMM tile shape.
constexpr int kGemmBM = 128;
constexpr int kGemmBN = 128;
constexpr int kGemmBK = 64;

// Runtime services shared by the C ABI's source files (runtime.hip).
// Records a message for vvh_last_error() and returns `status`.
int fail(int status, const char* fmt, ...);
// A fixed device buffer used as a call's workspace (split-K partial planes)
// in place of the per-stream workspace, which grows with hipMalloc.
struct WsSource {
    void* fixed = nullptr;
    std::size_t bytes = 0;
};
// vvh_linear_q8_dev with the workspace from wsrc (null: the stream's).
int linear_dev(void* out, const void* inp, const int8_t* w, const float* scales, const float* bias, const void* res,
               std::size_t M, std::size_t N, std::size_t K, int act, int outd, void* stream, const WsSource* wsrc);

// Launchers (linear_kernels.hip).  Return a hipError_t value as int.
int launch_generic(const LinArgs& a, int act, int out, void* stream);
int launch_gemv_f32(const LinArgs& a, int out, void* stream);
int launch_skinny(const LinArgs& a, int out, void* stream);
int launch_skinny_grouped(const LinArgs* dev_table, int count, int64_t total_blocks, int out,
                          void* stream);
// early: the variant for launches with few blocks, which requests the
// epilogue operands and the weight ring before staging the activations;
// depth: k steps in flight per wave (2, 4 or 7)
int launch_dot(const LinArgs& a, int out, bool early, int depth, void* stream);
// dev_block_prob[b] = problem of block b; args: the host copy of the
// count problems of dev_table (passed in the kernel arguments when count <=
// kDotInline); x_in_lds: dot_x_in_lds holds for every problem; lds_bytes =
// the largest dot_lds_bytes of the problems; pos: position of activation
// row 0 for problems with a RoPE epilogue
int launch_dot_grouped(const LinArgs* dev_table, const int32_t* dev_block_prob, const LinArgs* args, int count,
                       int64_t total_blocks, int max_m, bool x_in_lds, size_t lds_bytes, int out, bool early,
                       int depth, int64_t pos, void* stream);
int launch_gemm(const LinArgs& a, int out, void* stream);
// k_gemm3 (gemm_kernels.hip): one BM x BN tile (or one k split of it) per
// block, K % 64 == 0; layout 1 = 128 x 192, 3 = 128 x 128, 4 = 64 x 128
int gemm3_tile_n(int layout);
int gemm3_tile_m(int layout);
int launch_gemm3(const LinArgs& a, int out, int layout, void* stream);
// sum of the a.nsplit partials in a.ws + epilogue (scale, bias, residual)
int launch_splitk_reduce(const LinArgs& a, int out, void* stream);
// depth = weight loads in flight per lane (8 or 12); every problem must have
// at least `depth` 64-wide k steps.  max_m = largest M of the launch.
int launch_stream(const StreamArgs& s, int depth, int max_m, int out, int64_t blocks, void* stream);

// Model-step operators (model_kernels.hip); dtype = activation type
// (VVH_F32 / VVH_F16), computation in fp32.
int launch_eltwise(int op, void* out, const void* x, const void* y, int64_t n, int dtype, void* stream);
int launch_rms_norm(void* out, const void* x, const float* w, int64_t rows, int64_t n, float eps, int dtype,
                    void* stream);
int launch_softmax(void* out, const void* x, int64_t rows, int64_t n, int dtype, void* stream);
// out[i] = rope_freq(i, D, theta) for i < D / 2
int launch_rope_freq(float* out, int64_t D, float theta, void* stream);
// out[2 (p D / 2 + i)], out[2 (p D / 2 + i) + 1] = rope_cs_freq(p, freq[i])
// (cosine, sine) for p < positions, i < D / 2
int launch_rope_table(float* out, const float* freq, int64_t positions, int64_t D, void* stream);
int launch_rope(void* q, void* k, int64_t S, int64_t H, int64_t KVH, int64_t D, int64_t pos, float theta, int dtype,
                void* stream);
int launch_rope_append(void* q, void* k, const void* v, void* kc, void* vc, int64_t S, int64_t H, int64_t KVH,
                       int64_t D, int64_t pos, float theta, int dtype, void* stream);
int launch_embedding(void* out, const float* table, int64_t token, int64_t hidden, int dtype, void* stream);
int64_t attention_max_len();
int launch_attention(void* out, const void* q, const void* k, const void* v, int64_t n_q, int64_t len0, int64_t H,
                     int64_t KVH, int64_t D, float scale, int dtype, void* stream);
// n_q = 1 fast path: grouped heads, split over the sequence into nb blocks
// per kv head.  mfma: the fp16 matrix-core kernel (head_dim 64 or 128), which
// merges the blocks in the same launch and, with nb > 1, needs a zeroed
// arrival counter per kv head (cnt, kAttnCounters of them per stream); else
// the lane kernel, followed by a merge launch when nb > 1.  ws holds
// attention_decode_ws_floats() floats (none when nb == 1).
struct AttnDecodePlan {
    bool mfma;
    int waves;          // waves per block of the mfma kernel (4 or 8)
    int64_t per_block;  // keys per block
    int64_t nb;         // blocks per kv head
};
constexpr int64_t kAttnCounters = 16384;
bool attention_decode_ok(const void* k, const void* v, int64_t len, int64_t H, int64_t KVH, int64_t D);
int64_t attention_decode_max_len();
AttnDecodePlan attention_decode_plan(const void* q, int64_t len, int64_t H, int64_t KVH, int64_t D, int dtype);
int64_t attention_decode_ws_floats(const AttnDecodePlan& p, int64_t H, int64_t D);
inline bool attention_decode_counted(const AttnDecodePlan& p) { return p.mfma && p.nb > 1; }
int launch_attention_decode(const AttnDecodePlan& p, void* out, const void* q, const void* k, const void* v,
                            int64_t len, int64_t H, int64_t KVH, int64_t D, float scale, float* ws, unsigned* cnt,
                            int dtype, void* stream);
// Per-wave parts of the decode attention (k_attention_parts) for spans the
// matrix-core kernel takes in one block (mfma and nb == 1 in the plan);
// nparts = that block's waves.  parts: nparts * H rows of D + 4 floats.
int launch_attention_parts(float* parts, const void* q, const void* k, const void* v, int64_t len, int64_t H,
                           int64_t KVH, int64_t D, float scale, int nparts, void* stream);
int launch_zero_u32(unsigned* p, int64_t n, void* stream);
int launch_copy2(void* d0, const void* s0, void* d1, const void* s1, int64_t bytes, void* stream);
int launch_dense(void* out, const void* x, const void* w, int wdtype, const float* bias, const void* res, int64_t M,
                 int64_t N, int64_t K, int dtype, void* stream);
int launch_matmul(void* out, const void* A, const float* B, int64_t M, int64_t N, int64_t K, int dtype, void* stream);
// ws: argmax_ws_bytes(n) bytes (none for n <= 2048)
int64_t argmax_ws_bytes(int64_t n);
int launch_argmax(const float* x, int64_t n, int32_t* idx, float* ws, void* stream);
// temperature 0: argmax; > 0: Gumbel-max with the hash uniforms of (seed, step, i);
// x holds n values of dtype (VVH_F32 / VVH_F16); ws as for launch_argmax
int launch_sample(const void* x, int dtype, int64_t n, float temperature, uint64_t seed, int32_t step, int32_t* idx,
                  float* ws, void* stream);

// Auxiliary kernels (aux_kernels.hip).
// w: N x K elements of src_dtype (VVH_F32 or VVH_BF16)
int launch_quantize(const void* w, int src_dtype, int64_t N, int64_t K, int8_t* q, float* scales, void* stream);
int launch_convert(void* dst, int dst_dtype, const void* src, int src_dtype, int64_t n,
                   void* stream);
int launch_fill_normal(void* dst, int dtype, int64_t n, uint64_t seed, float mean, float std,
                       void* stream);
// fp32 rows x [M, K] -> xs [M, 2K] fp16 (scaled high parts, then low parts)
// and rs [M] (inverse scales), the activations of an fp32 call on the GEMM
int launch_split_f32(const float* x, int64_t M, int64_t K, void* xs, float* rs, void* stream);

}  // namespace vvh
