// k_gemm3: the prefill / batched int8 linear (fp16 activations, M > 16,
// K % 64 == 0), one output tile (or one k split of it) per block.
//
// out[M, N] = (x[M, K] . codes[N, K]^T) * scale[N] + bias[N] (+ res[M, N]),
// the Backend::linear_q8 / linear_q8_add contract
// (include/vvllm/backend/backend.h:62-65, 75-78) on MFMA.
//
// Block tile 128(m) x BN(n) x 64(k), BN = 32 * TJ * WN; (4 / TI) x WN waves,
// each a (32 * TI) x (32 * TJ) wave tile built from TI x TJ
// v_mfma_f32_32x32x16_f16 tiles.
// A wave tile trades LDS reads against code conversions: per MFMA a wave
// reads (TI * 4 KB of A + TJ * 2 KB of B) / (4 TI TJ) from LDS and converts
// 20 / TI codes' worth of VALU (5 ops per 4 codes, each converted fragment
// feeding TI row tiles).  64 x 96 (TI = 2, TJ = 3): 0.58 KB and 5 VALU per
// MFMA; 128 x 32 (TI = 4, TJ = 1): 1.25 KB and 2.5 VALU, which measured a
// few percent faster at 128 x 128 blocks.
//
// Operands are staged through a ring of D LDS stages filled by direct
// global -> LDS loads (global_load_lds_dwordx4), A as fp16 and B as the raw
// int8 codes, in the swizzled layout of swz_a / swz_b (device.h).  The
// codes are converted to fp16 exactly (two v_perm and one packed subtract
// per 4 codes) half a stage ahead of their MFMAs: the second k slice of a
// stage is converted during the first slice's MFMAs, and the first k slice
// of the next stage during the second slice's MFMAs, so no MFMA waits on a
// conversion once the loop runs.
//
// Step j (stage j in registers, its first slice converted):
//   wait for stage j+1's loads; barrier;
//   refill stage j's buffer with k stage j + D; read stage j+1's fragments;
//   MFMAs of (j, slice 0) || convert (j, slice 1);
//   MFMAs of (j, slice 1) || convert (j+1, slice 0).
// Stage indices, fragment parity and wait thresholds are compile-time
// constants (the loop is unrolled by D, D even).
//
// The MFMAs compute the transposed tile (codes as the A operand, activations
// as B): lane l then holds, for each group g of its 16 accumulator values,
// four consecutive outputs n of row m = l % 32, which go to LDS as one
// 16-byte write.
//
// Epilogue: the raw fp32 sums go through LDS (32-row quarter q of the tile
// in stage buffer q); each thread then owns one 8-wide column chunk (its 8
// scales and biases loaded at kernel start), applies acc * scale + bias
// (+ residual) in fp32 with one rounding, and stores rows with 16-byte
// non-temporal stores (the output is not read again by this kernel; measured
// M=2048 gate/up 30.8 -> 29.2 us against plain stores).  A tile wholly inside the problem (no split, N % 8 == 0) takes a
// branch-free path: its residual rows are loaded before the accumulators go
// to LDS, eight rows' LDS reads are in flight together and row addresses
// advance by a fixed stride (measured: 1.44 -> 0.72 us for the reads and
// stores of a 128 x 128 tile).  Edge tiles take the general path, four
// rows' LDS reads in flight at a time.
//
// Split-K (a.nsplit > 1, for few tiles over a long K): blocks enumerate
// (split, tile), tiles fastest; split ks runs k stages [ks * kstages,
// (ks + 1) * kstages) and writes its raw fp32 sums to ws[ks][M][N]; the
// reduction kernel then adds the splits in order and applies the epilogue.
#include "common.h"
#include "device.h"

namespace vvh
{

template <int BN, int BM>
struct Gemm3Stage {
    static constexpr int kOps = BM * kGemmBK * 2 + BN * kGemmBK;  // A fp16 + B codes
    static constexpr int kEpi = 32 * (BN + 4) * 4;                 // one 32-row epilogue quarter, fp32
    __attribute__((aligned(16))) f16 a[BM * kGemmBK];
    __attribute__((aligned(16))) int8_t b[BN * kGemmBK];
    __attribute__((aligned(16))) char pad[kEpi > kOps ? kEpi - kOps : 16];
};

template <int TJ, int TI>
struct Gemm3Frag {
    u4 b[2][TJ];      // raw codes: slice kk2, column tile tj
    h8 a[2][2][TI];   // fp16 A: slice kk2, half h, row tile ti
};

template <int TJ, int TI>
__device__ __forceinline__ void gemm3_read(const f16* __restrict__ sa, const int8_t* __restrict__ sb,
                                           Gemm3Frag<TJ, TI>& f, int row0, int col0, int fl, int fh)
{
#pragma unroll
    for (int kk2 = 0; kk2 < 2; kk2++) {
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            const int j = col0 + tj * 32 + fl;
            f.b[kk2][tj] = *reinterpret_cast<const u4*>(sb + j * 64 + swz_b(j, kk2 * 2 + fh) * 16);
        }
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int ti = 0; ti < TI; ti++) {
                const int i = row0 + ti * 32 + fl;
                f.a[kk2][h][ti] = *reinterpret_cast<const h8*>(sa + i * 64 + swz_a(i, kk2 * 4 + fh * 2 + h) * 8);
            }
    }
}

template <int TJ>
__device__ __forceinline__ void gemm3_convert(const u4 (&b)[TJ], h8 (&fb)[TJ][2])
{
#pragma unroll
    for (int tj = 0; tj < TJ; tj++) i8x16_to_h8x2(b[tj], fb[tj][0], fb[tj][1]);
}

// MFMAs of one 32-wide k slice (2 x TI x TJ of them) with the conversion of
// another slice's codes (20 * TJ VALU) spread between them.
template <int TJ, int TI>
__device__ __forceinline__ void gemm3_slice(const h8 (&a)[2][TI], const h8 (&fb)[TJ][2], f16v (&acc)[TI][TJ],
                                            const u4 (&nb)[TJ], h8 (&nfb)[TJ][2])
{
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int ti = 0; ti < TI; ti++)
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
                acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[tj][h], a[h][ti], acc[ti][tj], 0, 0, 0);
    gemm3_convert<TJ>(nb, nfb);
    constexpr int NM = 2 * TI * TJ;
    constexpr int NV = (20 * TJ + NM - 1) / NM;
#pragma unroll
    for (int i = 0; i < NM; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);  // then conversion VALU
    }
}

template <int TJ, int TI>
__device__ __forceinline__ void gemm3_slice_last(const h8 (&a)[2][TI], const h8 (&fb)[TJ][2], f16v (&acc)[TI][TJ])
{
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int ti = 0; ti < TI; ti++)
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
                acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[tj][h], a[h][ti], acc[ti][tj], 0, 0, 0);
}

// One stage's direct-to-LDS loads of this wave: buffer loads whose per-lane
// offsets are fixed for the whole k loop and whose stage offset k0 goes in
// the scalar offset, so a stage costs no address arithmetic.
template <int NW, int BN, int BM>
__device__ __forceinline__ void gemm3_fill(f16* __restrict__ sa, int8_t* __restrict__ sb, __amdgpu_buffer_rsrc_t ra,
                                           __amdgpu_buffer_rsrc_t rb, const uint32_t* a_off, const uint32_t* b_off,
                                           int wave, uint32_t ka, uint32_t kb)
{
    constexpr int LA = BM / 8 / NW, LB = BN / 16 / NW;
#pragma unroll
    for (int i = 0; i < LA; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, sa + (wave * LA + i) * 512, 16, a_off[i], ka * 2, 0, 0);
#pragma unroll
    for (int i = 0; i < LB; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, sb + (wave * LB + i) * 1024, 16, b_off[i], kb, 0, 0);
}

// BM = 64: blocks of half the LDS and registers, two resident per CU, so one
// block's MFMAs run while the other waits at its barrier or for its loads.
template <typename OT, int D, int WN, int TJ, int TI, int BM>
__global__ __launch_bounds__(64 * (BM / 32 / TI) * WN, BM == 64 ? 2 : 1) void k_gemm3(LinArgs a)
{
    static_assert(D == 4, "four stages: even (static fragment parity) and one epilogue quarter per stage");
    static_assert(TI == 2 || TI == 4, "wave tiles of 64 or 128 rows");
    static_assert(BM == 64 || BM == 128, "block tiles of 64 or 128 rows");
    constexpr int WM = BM / 32 / TI;  // waves along the BM rows
    static_assert(WM >= 1, "a wave tile within the block");
    constexpr int NW = WM * WN;
    constexpr int NT = 64 * NW;
    constexpr int BN = 32 * TJ * WN;
    static_assert((BM / 8) % NW == 0 && (BN / 16) % NW == 0, "whole 1 KB loads per wave");
    constexpr int LA = BM / 8 / NW, LB = BN / 16 / NW;
    constexpr int LPS = LA + LB;  // loads per stage per thread
    using Stage = Gemm3Stage<BN, BM>;
    using Frag = Gemm3Frag<TJ, TI>;
    __shared__ Stage st0, st1, st2, st3;

    const int64_t nbm = (a.M + BM - 1) / BM;
    const int64_t nbn = (a.N + BN - 1) / BN;
    const int64_t tiles = nbm * nbn;
    const bool split = a.nsplit > 1;
    // consecutive tiles (same n0, or same m0 with a.norder) on one XCD
    const int64_t logical = xcd_remap(blockIdx.x, tiles * (split ? a.nsplit : 1));
    const int64_t ks = logical / tiles, tile = logical - ks * tiles;
    const int64_t mb = a.norder ? tile / nbn : tile % nbm;
    const int64_t nb = a.norder ? tile - mb * nbn : tile / nbm;
    const int64_t m0 = mb * BM;
    const int64_t n0 = nb * BN;
    const int64_t kbase = split ? ks * a.kstages : 0;  // first k stage of this block

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int row0 = wm * (32 * TI), col0 = wn * (32 * TJ);
    const int fl = lane & 31, fh = lane >> 5;
    const f16* X = static_cast<const f16*>(a.inp);

    // epilogue: thread t < RG * CH owns column chunk t % CH (8 outputs) of
    // rows t / CH, t / CH + RG, ...; its scales and biases are loaded first
    // (the oldest loads in the vmcnt queue)
    constexpr int CH = BN / 8;
    constexpr int RG = NT / CH;
    const int ech = tid % CH, erg = tid / CH;
    const int64_t en = n0 + ech * 8;
    float sc[8], bi[8];
    if (split) {  // raw partial sums: the reduction applies the epilogue
#pragma unroll
        for (int e = 0; e < 8; e++) {
            sc[e] = 1.0f;
            bi[e] = 0.0f;
        }
    } else if (a.N % 8 == 0) {  // 16-byte loads at a clamped (always valid) chunk
        const int64_t ec = en < a.N ? en : a.N - 8;
        const f4 s0 = *reinterpret_cast<const f4*>(a.scales + ec), s1 = *reinterpret_cast<const f4*>(a.scales + ec + 4);
        f4 b0 = f4{}, b1 = f4{};
        if (a.bias) {
            b0 = *reinterpret_cast<const f4*>(a.bias + ec);
            b1 = *reinterpret_cast<const f4*>(a.bias + ec + 4);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            sc[e] = s0[e];
            sc[4 + e] = s1[e];
            bi[e] = b0[e];
            bi[4 + e] = b1[e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            sc[e] = en + e < a.N ? a.scales[en + e] : 0.0f;
            bi[e] = (a.bias && en + e < a.N) ? a.bias[en + e] : 0.0f;
        }
    }

    // buffer resources based at the tile's first row (rows past M or N read
    // the last valid row), per-lane byte offsets within them
    // KB: row length of the codes; a.bk != 0 (split fp32 activations, whose
    // rows hold K = 2 * KB values: hi parts, then lo parts) makes the code
    // stages wrap around at KB
    const int64_t KB = a.bk ? a.bk : a.K;
    const uint64_t a_bytes = (uint64_t)(a.M - m0) * a.K * 2, b_bytes = (uint64_t)(a.N - n0) * KB;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<f16*>(X + m0 * a.K), 0, (int)(a_bytes < 0xFFFFFFFFull ? a_bytes : 0xFFFFFFFFull), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(a.w + n0 * KB), 0, (int)(b_bytes < 0xFFFFFFFFull ? b_bytes : 0xFFFFFFFFull), 0x00020000);
    uint32_t a_off[LA];
#pragma unroll
    for (int i = 0; i < LA; i++) {
        const int r = (wave * LA + i) * 8 + (lane >> 3);
        const int64_t gr = m0 + r < a.M ? r : a.M - 1 - m0;
        a_off[i] = (uint32_t)(gr * a.K * 2 + swz_a(r, lane & 7) * 16);
    }
    uint32_t b_off[LB];
#pragma unroll
    for (int i = 0; i < LB; i++) {
        const int r = (wave * LB + i) * 16 + (lane >> 2);
        const int64_t gn = n0 + r < a.N ? r : a.N - 1 - n0;
        b_off[i] = (uint32_t)(gn * KB + swz_b(r, lane & 3) * 16);
    }

    auto stage = [&](auto S) -> Stage& {
        constexpr int s = decltype(S)::value % D;
        if constexpr (s == 0) return st0;
        else if constexpr (s == 1) return st1;
        else if constexpr (s == 2) return st2;
        else return st3;
    };
    auto issue = [&](Stage& g, int64_t kt) {
        const int64_t k0 = (kbase + kt) * kGemmBK;
        gemm3_fill<NW, BN, BM>(g.a, g.b, ra, rb, a_off, b_off, wave, (uint32_t)k0, (uint32_t)(k0 < KB ? k0 : k0 - KB));
    };

    f16v acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++) acc[i][j] = f16v{};
    Frag f0, f1;
    h8 fb[2][TJ][2];  // converted codes: slice, column tile, half
    auto frag = [&](auto P) -> Frag& {
        if constexpr (decltype(P)::value % 2 == 0) return f0;
        else return f1;
    };
    auto read = [&](auto S) { gemm3_read<TJ, TI>(stage(S).a, stage(S).b, frag(S), row0, col0, fl, fh); };

    // one step of the schedule; NEXT: stage j+1 exists, REFILL: refill
    // stage j's buffer with k stage kt0 + j + D, VM: loads still allowed in
    // flight once stage j+1 has landed
    auto step = [&]<int J, bool NEXT, bool REFILL, int VM>(int64_t kt0) {
        constexpr auto j = std::integral_constant<int, J>{};
        constexpr auto jn = std::integral_constant<int, J + 1>{};
        if constexpr (NEXT) wait_vmcnt<VM>();
        lds_barrier();
        if constexpr (REFILL) issue(stage(j), kt0 + J + D);
        if constexpr (NEXT) read(jn);
        Frag& f = frag(j);
        gemm3_slice<TJ, TI>(f.a[0], fb[0], acc, f.b[1], fb[1]);
        if constexpr (NEXT) gemm3_slice<TJ, TI>(f.a[1], fb[1], acc, frag(jn).b[0], fb[0]);
        else gemm3_slice_last<TJ, TI>(f.a[1], fb[1], acc);
    };
    // R steps from kt0 (kt0 % D == 0) with the problem's stage count kt0 + R
    auto steps = [&]<int R>(int64_t kt0) {
        [&]<int... J>(std::integer_sequence<int, J...>) {
            (step.template operator()<J, (J + 1 < R), (J + D < R),
                                      ((R - 2 - J < D - 2) ? R - 2 - J : D - 2) * LPS>(kt0),
             ...);
        }(std::make_integer_sequence<int, R>{});
    };
    auto prologue = [&]<int P>() {
        [&]<int... S>(std::integer_sequence<int, S...>) {
            (issue(stage(std::integral_constant<int, S>{}), S), ...);
        }(std::make_integer_sequence<int, P>{});
        wait_vmcnt<(P - 1) * LPS>();
        lds_barrier();
        read(std::integral_constant<int, 0>{});
        gemm3_convert<TJ>(f0.b[0], fb[0]);
    };

    const int64_t nk_all = a.K / kGemmBK;
    const int64_t nk = split ? (nk_all - kbase < a.kstages ? nk_all - kbase : a.kstages) : nk_all;
    if (nk >= D) {
        prologue.template operator()<D>();
        int64_t kt0 = 0;
        for (; kt0 + 2 * D <= nk; kt0 += D) {
            // a full group: every step refills and waits at the steady-state depth
            [&]<int... J>(std::integer_sequence<int, J...>) {
                (step.template operator()<J, true, true, (D - 2) * LPS>(kt0), ...);
            }(std::make_integer_sequence<int, D>{});
        }
        const int64_t r = nk - kt0;  // D .. 2D-1
        [&]<int... R>(std::integer_sequence<int, R...>) {
            ((r == R + D ? steps.template operator()<R + D>(kt0) : void()), ...);
        }(std::make_integer_sequence<int, D>{});
    } else {
        [&]<int... R>(std::integer_sequence<int, R...>) {
            ((nk == R + 1 ? [&] {
                prologue.template operator()<R + 1>();
                steps.template operator()<R + 1>(0);
            }() : void()), ...);
        }(std::make_integer_sequence<int, D - 1>{});
    }

    // ---- epilogue ----
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    constexpr int ES = BN + 4;  // fp32 row stride of an epilogue quarter
    auto quarter = [&](int q) -> float* {
        return reinterpret_cast<float*>(q == 0 ? &st0 : q == 1 ? &st1 : q == 2 ? &st2 : &st3);
    };
    constexpr int RI = (BM + RG - 1) / RG;  // rows per thread
    // Interior tiles (every row and column inside the problem, whole 8-wide
    // chunks, no split) take a branch-free path; its residual rows are
    // loaded here, so their latency overlaps the accumulator transpose.
    const bool interior = !split && m0 + BM <= a.M && n0 + BN <= a.N && a.N % 8 == 0;
    const bool own = erg < RG;
    constexpr int RW = sizeof(OT) / 2;  // 16-byte chunks per 8 outputs
    u4 rr[RI][RW];
    const int64_t o_first = (m0 + erg) * a.N + en, o_step = RG * a.N;
    if (interior && own && a.res) {
        const OT* rp = static_cast<const OT*>(a.res) + o_first;
#pragma unroll
        for (int i = 0; i < RI; i++)
            if (i + 1 < RI || erg + i * RG < BM)
#pragma unroll
                for (int c = 0; c < RW; c++) rr[i][c] = reinterpret_cast<const u4*>(rp + i * o_step)[c];
    }
    if (a.xrs) {
        // split fp32 activations: each row's sums times its power-of-two scale
#pragma unroll
        for (int ti = 0; ti < TI; ti++) {
            const int64_t m = m0 + row0 + ti * 32 + fl;
            const float rs = a.xrs[m < a.M ? m : a.M - 1];
#pragma unroll
            for (int tj = 0; tj < TJ; tj++) acc[ti][tj] *= rs;
        }
    }
#pragma unroll
    for (int ti = 0; ti < TI; ti++) {
        float* q = quarter((row0 >> 5) + ti) + fl * ES + col0 + 4 * fh;
#pragma unroll
        for (int tj = 0; tj < TJ; tj++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *reinterpret_cast<f4*>(q + tj * 32 + 8 * g) =
                    f4{acc[ti][tj][4 * g], acc[ti][tj][4 * g + 1], acc[ti][tj][4 * g + 2], acc[ti][tj][4 * g + 3]};
    }
    lds_barrier();
    if (!own) return;
    // lanes 8-15 of a 16-lane read group take the other half of their chunk
    // first, so the group covers distinct banks
    const int sw = (ech >> 3) & 1;
    if (interior) {
        constexpr int UB = 8;  // rows whose LDS reads are in flight together
#pragma unroll
        for (int i0 = 0; i0 < RI; i0 += UB) {
            f4 p[UB], q[UB];
#pragma unroll
            for (int u = 0; u < UB; u++) {
                const int i = i0 + u, row = erg + i * RG;
                if (i < RI && (i + 1 < RI || row < BM)) {
                    const float* tq = quarter(row >> 5) + (row & 31) * ES + ech * 8;
                    p[u] = *reinterpret_cast<const f4*>(tq + 4 * sw);
                    q[u] = *reinterpret_cast<const f4*>(tq + 4 - 4 * sw);
                }
            }
#pragma unroll
            for (int u = 0; u < UB; u++) {
                const int i = i0 + u, row = erg + i * RG;
                if (!(i < RI && (i + 1 < RI || row < BM))) continue;
                const f4 lo = sw ? q[u] : p[u], hi = sw ? p[u] : q[u];
                float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = v[e] * sc[e] + bi[e];
                OT* op = static_cast<OT*>(a.out) + o_first + i * o_step;
                if constexpr (sizeof(OT) == 2) {
                    if (a.res) {
                        const h8 r8 = __builtin_bit_cast(h8, rr[i][0]);
#pragma unroll
                        for (int e = 0; e < 8; e++) v[e] += (float)r8[e];
                    }
                    h8 o8;
#pragma unroll
                    for (int e = 0; e < 8; e++) o8[e] = (f16)v[e];
                    __builtin_nontemporal_store(o8, reinterpret_cast<h8*>(op));
                } else {
                    if (a.res) {
                        const f4 r0 = __builtin_bit_cast(f4, rr[i][0]), r1 = __builtin_bit_cast(f4, rr[i][1]);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            v[e] += r0[e];
                            v[e + 4] += r1[e];
                        }
                    }
                    __builtin_nontemporal_store(f4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f4*>(op));
                    __builtin_nontemporal_store(f4{v[4], v[5], v[6], v[7]}, reinterpret_cast<f4*>(op + 4));
                }
            }
        }
        return;
    }
    if (en >= a.N) return;
    const bool vec = (a.N % 8) == 0 && en + 8 <= a.N;
    constexpr int U = 4;  // rows whose LDS reads are in flight together
#pragma unroll
    for (int i0 = 0; i0 < RI; i0 += U) {
        f4 v0[U], v1[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int row = erg + (i0 + u) * RG;
            if (i0 + u < RI && row < BM) {
                const float* tq = quarter(row >> 5) + (row & 31) * ES + ech * 8;
                const f4 p = *reinterpret_cast<const f4*>(tq + 4 * sw);
                const f4 q = *reinterpret_cast<const f4*>(tq + 4 - 4 * sw);
                v0[u] = sw ? q : p;
                v1[u] = sw ? p : q;
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int row = erg + (i0 + u) * RG;
            const int64_t mm = m0 + row;
            if (!(i0 + u < RI && row < BM) || mm >= a.M) continue;
            float v[8] = {v0[u][0], v0[u][1], v0[u][2], v0[u][3], v1[u][0], v1[u][1], v1[u][2], v1[u][3]};
            const int64_t o = mm * a.N + en;
            if (split) {  // raw partial sums of this split
                float* wp = a.ws + ks * a.M * a.N + o;
                if (vec) {
                    *reinterpret_cast<f4*>(wp) = v0[u];
                    *reinterpret_cast<f4*>(wp + 4) = v1[u];
                } else {
                    for (int e = 0; e < 8 && en + e < a.N; e++) wp[e] = v[e];
                }
                continue;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = v[e] * sc[e] + bi[e];
            if (vec) {
                if constexpr (sizeof(OT) == 2) {
                    if (a.res) {
                        const h8 r8 = *reinterpret_cast<const h8*>(static_cast<const f16*>(a.res) + o);
#pragma unroll
                        for (int e = 0; e < 8; e++) v[e] += (float)r8[e];
                    }
                    h8 o8;
#pragma unroll
                    for (int e = 0; e < 8; e++) o8[e] = (f16)v[e];
                    __builtin_nontemporal_store(o8, reinterpret_cast<h8*>(static_cast<f16*>(a.out) + o));
                } else {
                    if (a.res) {
                        const f4 r0 = *reinterpret_cast<const f4*>(static_cast<const float*>(a.res) + o);
                        const f4 r1 = *reinterpret_cast<const f4*>(static_cast<const float*>(a.res) + o + 4);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            v[e] += r0[e];
                            v[e + 4] += r1[e];
                        }
                    }
                    __builtin_nontemporal_store(f4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f4*>(static_cast<float*>(a.out) + o));
                    __builtin_nontemporal_store(f4{v[4], v[5], v[6], v[7]},
                                                reinterpret_cast<f4*>(static_cast<float*>(a.out) + o + 4));
                }
            } else {
                for (int e = 0; e < 8 && en + e < a.N; e++) {
                    float x = v[e];
                    if (a.res) x += ld_f(static_cast<const OT*>(a.res) + o + e);
                    st_f(static_cast<OT*>(a.out) + o + e, x);
                }
            }
        }
    }
}

// Tile shapes (layout code -> WN, TJ, TI, BM): 1 = 128 x 192 (4 waves of
// 64 x 96), 3 = 128 x 128 (4 waves of 128 x 32: each converted code
// fragment feeds 4 row tiles, 2.5 conversion VALU per MFMA; measured against
// 4 waves of 64 x 64 in the same runs: M=512 gate/up 11.13 -> 10.78 us,
// M=2048 33.7 -> 33.3 us, split-K down M=2048 32.7 -> 32.0 us), 4 = 64 x 128
// (4 waves of 64 x 32, two blocks per CU), 5 = 64 x 64 (2 waves of 64 x 32:
// a block fills 12 KB of LDS per stage instead of 16, for calls whose 64 x 64
// tiles, or split tiles, fit one round over the CUs).
int gemm3_tile_n(int layout) { return layout == 1 ? 192 : layout == 5 ? 64 : 128; }
int gemm3_tile_m(int layout) { return (layout == 4 || layout == 5) ? 64 : 128; }

template <int WN, int TJ, int TI, int BM>
static void gemm3_go(const LinArgs& a, bool f32, hipStream_t s)
{
    constexpr int BN = 32 * TJ * WN;
    constexpr int NT = 64 * (BM / 32 / TI) * WN;
    const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const dim3 grid((unsigned)(tiles * (a.nsplit > 1 ? a.nsplit : 1)));
    if (f32) hipLaunchKernelGGL((k_gemm3<float, 4, WN, TJ, TI, BM>), grid, dim3(NT), 0, s, a);
    else hipLaunchKernelGGL((k_gemm3<f16, 4, WN, TJ, TI, BM>), grid, dim3(NT), 0, s, a);
}

int launch_gemm3(const LinArgs& a, int out, int layout, void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool f32 = out == VVH_F32;
    if (layout == 3) gemm3_go<4, 1, 4, 128>(a, f32, s);
    else if (layout == 4) gemm3_go<4, 1, 2, 64>(a, f32, s);
    else if (layout == 5) gemm3_go<2, 1, 2, 64>(a, f32, s);
    else gemm3_go<2, 3, 2, 128>(a, f32, s);
    return (int)hipGetLastError();
}

}  // namespace vvh
