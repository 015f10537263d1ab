/*
 * vvllm_hip.h -- C ABI of the MI355X (gfx950) INT8 per-channel linear path.
 *
 * This is the drop-in boundary that sits under a vvllm `Backend`
 * implementation (see vvllm_amd/host/backend_hip.h): plain pointers, sizes
 * and integer status codes, no C++ or HIP types in any signature.  Each entry
 * names the reference interface it replaces (paths relative to the vvllm
 * source tree).  In the reference those functions return void and call
 * exit(1) on any CUDA error (src/backend/cuda_kernels.cu:11-21); here every
 * entry returns a vvh_status and never exits.
 *
 * Conventions
 *   - "device pointer" = memory from vvh_malloc / vvh_pool_alloc (or any
 *     HIP device allocation); "host pointer" = ordinary CPU memory.
 *   - Weights are [N, K] row-major int8 codes with per-row fp32 scales
 *     (the QuantizedWeight layout, include/vvllm/quantize/quantize.h:10-14).
 *   - Activations are [M, K] row-major, outputs and residuals [M, N]
 *     row-major, in the dtype given by act_dtype / out_dtype.
 *   - `stream` is a hipStream_t passed as void*; NULL = the null stream.
 *     Launches are asynchronous on it; errors of the launch itself are
 *     reported, errors of the kernel's execution surface at the next
 *     synchronising call.
 *   - Split-K GEMMs, fp32-activation GEMMs (M * K * 4 + M * 4 bytes for the
 *     split activations), multi-chunk decode attention and multi-block
 *     sampling use a per-stream workspace that grows on demand (hipMalloc, to at
 *     least twice its size, never below 1 MiB).  Under HIP graph capture it
 *     cannot grow: run the same calls once on that stream before capturing
 *     (decode attention needs at most 512 * (num_heads / num_kv_heads) *
 *     (head_dim + 2) * 4 bytes, 4.3 MB, at any span).  A buffer the
 *     workspace outgrows is kept, not freed, so graphs captured before the
 *     growth stay valid; vvh_workspace_release frees them all.
 *   - All calls may be made from one host thread at a time per device
 *     (as the reference, which is single-threaded, README.md:282); the
 *     allocator and registries are internally locked.
 */
#ifndef VVLLM_HIP_H
#define VVLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define VVH_API __attribute__((visibility("default")))
#else
#define VVH_API
#endif

/* ---- status codes ---------------------------------------------------- */
typedef enum vvh_status {
    VVH_OK = 0,
    VVH_ERR_INVALID_ARG = 1,      /* null pointer, bad dtype, size overflow, ... */
    VVH_ERR_NO_DEVICE = 2,        /* no HIP device / bad device index */
    VVH_ERR_OUT_OF_MEMORY = 3,    /* device allocation failed after cache release */
    VVH_ERR_HIP = 4,              /* any other HIP runtime error */
    VVH_ERR_NOT_INITIALIZED = 5,  /* vvh_init has not succeeded yet */
    VVH_ERR_UNKNOWN_HANDLE = 6,   /* weight / plan handle not registered */
    VVH_ERR_UNSUPPORTED = 7,      /* valid call the library cannot serve */
} vvh_status;

/* Element types: activations, outputs and residuals are F32 or F16;
 * weights handed to vvh_weight_ingest are F32 or BF16. */
typedef enum vvh_dtype {
    VVH_F32 = 0,
    VVH_F16 = 1,
    VVH_BF16 = 2,
} vvh_dtype;

/* Human-readable name of a status code (static storage). */
VVH_API const char* vvh_status_string(int status);
/* Message describing the most recent failure on the calling thread
 * (empty string if none).  Valid until the next failing call. */
VVH_API const char* vvh_last_error(void);
/* Library version string, e.g. "vvllm-hip 0.1 gfx950". */
VVH_API const char* vvh_version(void);

/* ---- device ------------------------------------------------------------ */
/* Selects HIP device `device` for this process and writes its name.
 * Replaces cuda_init_device (src/backend/cuda_kernels.h:21-22,
 * src/backend/cuda_kernels.cu:583-595), which exits the process when no
 * device is present; this returns VVH_ERR_NO_DEVICE instead. */
VVH_API int vvh_init(int device, char* name_buf, size_t name_buf_size);
/* Waits for all work on the device.  Replaces cuda_sync
 * (src/backend/cuda_kernels.h:19). */
VVH_API int vvh_sync(void);
/* Number of compute units of the current device (0 before vvh_init). */
VVH_API int vvh_device_cu_count(void);

/* ---- raw device memory ------------------------------------------------ */
/* Replace cuda_malloc / cuda_free / cuda_malloc_host / cuda_free_host /
 * cuda_memcpy_{h2d,d2h,d2d} (src/backend/cuda_kernels.h:11-17,
 * src/backend/cuda_kernels.cu:543-579).  Copies are synchronous, as there. */
VVH_API int vvh_malloc(void** ptr, size_t bytes);
VVH_API int vvh_free(void* ptr);
VVH_API int vvh_malloc_host(void** ptr, size_t bytes);
VVH_API int vvh_free_host(void* ptr);
VVH_API int vvh_memcpy_h2d(void* dst, const void* src, size_t bytes);
VVH_API int vvh_memcpy_d2h(void* dst, const void* src, size_t bytes);
VVH_API int vvh_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Device-to-device copy queued on `stream` (not synchronous): the KV-cache
 * append of a decode step (KVCacheCUDA::append copies synchronously,
 * src/kv_cache/kv_cache_cuda.cc:74-79). */
VVH_API int vvh_memcpy_d2d_async(void* dst, const void* src, size_t bytes, void* stream);
/* The KV-cache append's two device-to-device copies (k rows and v rows,
 * `bytes` each; KVCacheCUDA::append, src/kv_cache/kv_cache_cuda.cc:40-79)
 * as one kernel queued on `stream`.  Source and destination ranges must not
 * overlap. */
VVH_API int vvh_kv_append(void* k_dst, void* v_dst, const void* k_src, const void* v_src, size_t bytes, void* stream);

/* Frees the workspace of `stream` and every buffer it outgrew, after waiting
 * for the device.  Graphs captured on that stream that use the workspace
 * must not be replayed afterwards (the next call that needs it allocates a
 * new one).  No reference counterpart (the reference has no workspace). */
VVH_API int vvh_workspace_release(void* stream);

/* ---- caching allocator -------------------------------------------------- */
/* Stream-ordered-free caching allocator behind device_allocate /
 * device_deallocate for the GPU device.  Replaces cuda_pool_alloc /
 * cuda_pool_free and the CUDA branch of device_allocate / device_deallocate
 * (src/tensor/tensor.cc:35-68, :72-96).  Unlike the reference's exact-size
 * free list it rounds requests to size classes, reuses best-fit cached
 * blocks, and on a failed hipMalloc returns every cached block to the
 * driver and retries once before reporting VVH_ERR_OUT_OF_MEMORY.
 * vvh_pool_alloc(&p, 0) yields p = NULL (as device_allocate, tensor.cc:74). */
VVH_API int vvh_pool_alloc(void** ptr, size_t bytes);
/* Returns a block to the cache.  Pointers that did not come from the pool
 * are freed with hipFree, as tensor.cc:58-66 does.  NULL is a no-op. */
VVH_API int vvh_pool_free(void* ptr);
/* hipFree every cached (free) block. */
VVH_API int vvh_pool_release_cached(void);

typedef struct vvh_pool_stats {
    uint64_t bytes_in_use;      /* rounded bytes handed out and not yet freed */
    uint64_t bytes_cached;      /* rounded bytes held in the free lists */
    uint64_t bytes_reserved;    /* bytes_in_use + bytes_cached */
    uint64_t peak_reserved;
    uint64_t alloc_calls;
    uint64_t cache_hits;        /* allocations served without hipMalloc */
    uint64_t driver_allocs;     /* hipMalloc calls made by the pool */
    uint64_t oom_releases;      /* times the cache was flushed to satisfy a request */
} vvh_pool_stats;
VVH_API int vvh_pool_get_stats(vvh_pool_stats* out);

/* ---- weight mirror ------------------------------------------------------ */
/* Device-resident copy of one quantized weight (codes + scales + optional
 * bias), uploaded once.  Replaces BackendCUDA::cache_weight /
 * cache_weight_fp16 (src/backend/backend_cuda.cc:51-77) and the
 * int8->fp16 dequantisation it triggers (src/backend/cuda_kernels.cu:804-814,
 * :833-840): the mirror keeps the raw int8 codes (1 byte/weight, not the
 * reference's int8 + fp16 = 3 bytes) and scales are applied in the kernels'
 * epilogue.
 *
 * The reference keys its cache by host address only, forever, so a freed and
 * reused host buffer would hit a stale copy.  Here the key is the full tuple
 * (weight ptr, scales ptr, bias ptr, N, K); registering an existing host
 * weight pointer with a different tuple replaces (frees and re-uploads) the
 * old mirror.  vvh_weight_release drops a mirror explicitly.
 * Handles are never 0. */
typedef uint64_t vvh_weight;
VVH_API int vvh_weight_register(const int8_t* host_weight, const float* host_scales,
                                const float* host_bias, size_t N, size_t K,
                                vvh_weight* handle);
/* Same, for codes/scales/bias already in device memory (not copied, not
 * owned: the caller keeps them alive until vvh_weight_release). */
VVH_API int vvh_weight_register_device(const int8_t* dev_weight, const float* dev_scales,
                                       const float* dev_bias, size_t N, size_t K,
                                       vvh_weight* handle);
/* Weight ingestion: quantizes the host weight rows `host_weight` (N x K
 * elements of src_dtype, VVH_F32 or VVH_BF16, row-major: e.g. a tensor of an
 * mmap'ed safetensors file) straight into a new device mirror.  The rows go
 * to the device in their stored width (2 bytes per BF16 weight), are widened
 * to fp32 in registers (exact: BF16 bits are the high half of the fp32, as in
 * the reference loader, src/safetensors/safetensors.cc:112-119, :135-141) and
 * quantized by the device quantizer, so codes and scales are bit-identical to
 * the host path it replaces: widen to fp32 on the host, then
 * quantize_per_channel (src/model/qwen2/model.cc:27-33,
 * src/quantize/quantize.cc:9-48).  The N scales are also written to
 * host_scales.  host_bias (F32, optional) is mirrored as with
 * vvh_weight_register.
 * The mirror is keyed by the tuple (host_weight, host_scales, host_bias, N, K):
 * a later vvh_weight_register / vvh_linear_q8 with host_weight reinterpreted
 * as the int8 pointer and the same scales/bias pointers finds it, so
 * Backend::linear_q8 callers can pass the ingested rows' address as the
 * weight.  Synchronous.  Uses two 32 MB pinned host staging buffers and two
 * device ones, allocated on the first call and kept until the process ends. */
VVH_API int vvh_weight_ingest(const void* host_weight, int src_dtype, const float* host_bias, size_t N,
                              size_t K, float* host_scales, vvh_weight* handle);
/* Finds the mirror of a host weight pointer; VVH_ERR_UNKNOWN_HANDLE if none. */
VVH_API int vvh_weight_find(const int8_t* host_weight, vvh_weight* handle);
VVH_API int vvh_weight_release(vvh_weight handle);
/* Device pointers of a mirror (bias NULL if it has none). */
VVH_API int vvh_weight_device_ptrs(vvh_weight handle, const int8_t** dev_weight,
                                   const float** dev_scales, const float** dev_bias,
                                   size_t* N, size_t* K);
/* Number of live mirrors and their total device bytes. */
VVH_API int vvh_weight_stats(uint64_t* count, uint64_t* bytes);

/* ---- the linear path ---------------------------------------------------- */
/* out[M,N] = (inp[M,K] . weight[N,K]^T) * scales[N] + bias[N] (+ residual[M,N])
 *
 * Replaces Backend::linear_q8 / linear_q8_add
 * (include/vvllm/backend/backend.h:62-65, :75-78) as implemented by
 * BackendCUDA (src/backend/backend_cuda.cc:188-213, :246-275) and the
 * unused cuda_linear_q8 / cuda_linear_q8_add launchers
 * (src/backend/cuda_kernels.h:25-26, :51-52).
 *   - inp, out, residual: device pointers of act_dtype / out_dtype /
 *     out_dtype; residual may be NULL; out == residual is allowed (the
 *     in-place residual connection of include/vvllm/model/transformer.h:
 *     165-166, 187-188).  Any other overlap of out with inp is undefined.
 *   - The dot product is accumulated in fp32 from the exact int8 codes;
 *     fp16 activations are used as given (no re-rounding).  fp32
 *     activations are not rounded to fp16 as the reference's CUDA fp32 mode
 *     does (backend_cuda.cc:205-211): the decode kernels (M < 16, or
 *     K % 64 != 0) use them as they are; the GEMM (M >= 16) multiplies each
 *     row, scaled by a power of two, as a pair of fp16 values (high part,
 *     then the exact remainder rounded to fp16), about 22 significant bits
 *     of each activation, with exact products and fp32 accumulation.
 *   - Epilogue in fp32, one rounding to out_dtype:
 *     out = acc*scale + bias + residual.
 *   - M == 0 or N == 0 is a no-op; K == 0 gives bias (+ residual). */
VVH_API int vvh_linear_q8(void* out, const void* inp, vvh_weight weight, const void* residual,
                          size_t M, size_t N, size_t K, int act_dtype, int out_dtype,
                          void* stream);
/* Same, with the weight given as device pointers (bias may be NULL). */
VVH_API int vvh_linear_q8_dev(void* out, const void* inp, const int8_t* dev_weight,
                              const float* dev_scales, const float* dev_bias,
                              const void* residual, size_t M, size_t N, size_t K,
                              int act_dtype, int out_dtype, void* stream);

/* Size of the fixed device scratch of vvh_linear_q8_dev_noalloc.  One call
 * needs the split-K partial planes (M * N * 4 bytes per split; on a 256-CU
 * device the dispatcher splits only GEMMs of at most 128 output tiles of
 * 64 x 128, into at most 256 blocks: at most 256 fp32 tiles of 32 KiB =
 * 8 MiB) plus, for fp32 activations on the GEMM (M >= 16), their split fp16
 * form: M * K * 4 bytes and M * 4 bytes, each rounded up to 256.  32 MiB
 * holds every fp16-activation call and fp32-activation calls up to about
 * 6 M activation elements (the configs[3] shapes in fp32 up to M = 1024 at
 * K = 4864, e.g. the down projection at M = 512: 9.96 MB + 4 planes of
 * 1.84 MB); a call that needs more returns VVH_ERR_UNSUPPORTED before any
 * launch (vvh_linear_q8_dev runs it). */
#define VVH_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
/* vvh_linear_q8_dev that allocates nothing: same arguments, same kernels and
 * the same result bits as vvh_linear_q8_dev, but the split-K partial planes
 * go to a fixed VVH_NOALLOC_SCRATCH_BYTES device array that the library
 * holds on each device from vvh_init until the process ends, instead of the
 * stream's workspace (which grows with hipMalloc); so do the split
 * activations of an fp32-activation GEMM (M >= 16: M * K * 4 + M * 4 bytes).
 * No hipMalloc, hipFree or allocating library routine is called.  A call
 * whose workspace needs more than VVH_NOALLOC_SCRATCH_BYTES (the bound above)
 * returns VVH_ERR_UNSUPPORTED and launches nothing.
 * No counterpart in the reference; for callers that cannot allocate: code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  All calls on one device share the one array, so calls that
 * overlap in time on that device (different streams, or threads) race;
 * calls queued in order on one stream do not. */
VVH_API int vvh_linear_q8_dev_noalloc(void* out, const void* inp, const int8_t* dev_weight,
                                      const float* dev_scales, const float* dev_bias,
                                      const void* residual, size_t M, size_t N, size_t K,
                                      int act_dtype, int out_dtype, void* stream);

/* Input stages of a decode linear (no counterpart in the reference, whose
 * transformer_forward runs the operator before the linear as its own call,
 * transformer.h:133-139, 176-185).  The linear reads its activation rows
 * through the stage, with the same arithmetic and fp16 rounding as the
 * standalone operator, and runs on the k_dot family (VVH_KERNEL_DOT), so the
 * result equals the operator followed by vvh_linear_q8_dev on that family
 * exactly (the automatic choice for M <= 2, and for M <= 8 below 1024
 * 16-row tiles). */
enum {
    VVH_IN_NONE = 0,
    VVH_IN_RMS_NORM = 1,  /* rows of inp -> vvh_rms_norm(in_w, in_eps) (:68-76) */
    VVH_IN_SILU_MUL = 2,  /* rows of inp are [gate | up] of 2K values -> silu(gate) * up (:293-300) */
};
/* vvh_linear_q8_dev of the staged input.  Stages other than VVH_IN_NONE need
 * fp16 activations, M <= 4, K % 16 == 0, 16-byte aligned inp, weights and
 * in_w (fp32 [K], RMSNorm only), and M rows of K + 8 halves within the
 * decode kernel's 80 KB of LDS; otherwise VVH_ERR_UNSUPPORTED.  For
 * VVH_IN_SILU_MUL, inp holds M rows of 2K values (gate, then up). */
VVH_API int vvh_linear_q8_dev_in(void* out, const void* inp, const int8_t* dev_weight,
                                 const float* dev_scales, const float* dev_bias,
                                 const void* residual, size_t M, size_t N, size_t K,
                                 int act_dtype, int out_dtype, int in_op, const float* in_w,
                                 float in_eps, void* stream);

/* ---- grouped launch ------------------------------------------------------ */
/* A plan is a fixed list of independent linear_q8 problems of one
 * (act_dtype, out_dtype) pair, resolved once (kernel choice, tile
 * decomposition, device-resident descriptor table) and launched with
 * vvh_plan_run as a single kernel when every problem takes the decode path
 * (M <= 16), else as one launch per problem.  It is the counterpart of the
 * reference IR's pre-resolved op list (src/ir/executable.cc:192-354) for the
 * int8 linears that share an input (q/k/v, transformer.h:139-144) or are
 * otherwise independent.  Problems must not write memory another problem of
 * the same plan reads. */
typedef struct vvh_q8_problem {
    void* out;
    const void* inp;
    const void* residual;      /* may be NULL */
    const int8_t* weight;      /* device */
    const float* scales;       /* device */
    const float* bias;         /* device, may be NULL */
    uint64_t M, N, K;
} vvh_q8_problem;
typedef uint64_t vvh_plan;
VVH_API int vvh_plan_create(const vvh_q8_problem* problems, size_t count, int act_dtype,
                            int out_dtype, vvh_plan* plan);
VVH_API int vvh_plan_run(vvh_plan plan, void* stream);
VVH_API int vvh_plan_destroy(vvh_plan plan);
/* Number of kernel launches one vvh_plan_run makes. */
VVH_API int vvh_plan_launches(vvh_plan plan, int* launches);
/* Gives every problem of a plan the input stage in_op (VVH_IN_*, with
 * in_w / in_eps as for vvh_linear_q8_dev_in): e.g. q/k/v reading the
 * residual stream through the layer's input RMSNorm.  The plan must run as
 * one k_dot_grouped launch with its activations in LDS (vvh_plan_kernel
 * gives VVH_KERNEL_DOT), else VVH_ERR_UNSUPPORTED.  The stage is written
 * into the plan's device table in place, after waiting for the device
 * (queued runs of the plan read that table): set it before capturing any
 * graph that runs the plan.  A graph captured before the call is not
 * updated (a plan of up to 4 problems passes its table in each launch's
 * kernel arguments): capture it again.  Calling it while a stream is being
 * captured fails (it synchronises the device). */
VVH_API int vvh_plan_set_input_op(vvh_plan plan, int in_op, const float* in_w, float in_eps);
/* RoPE and the KV-cache append as the epilogue of a q/k/v plan: problems
 * q_index, k_index and v_index (indices into the list given to
 * vvh_plan_create) then write what vvh_rope_append would leave after a plain
 * run of the plan, bit for bit: q and k rotated in place (split-half RoPE of
 * each head of head_dim, base theta, at position pos + m for activation row
 * m), and the rotated k rows and the v rows also written to rows pos + m of
 * k_cache and v_cache ([*, N of k] of the plan's output dtype).  Saves the
 * RoPE launch of a decode layer (transformer.h:145-160, the reference's
 * rope then KVCache::append).  No reference counterpart.  The plan must run
 * as one k_dot_grouped launch (vvh_plan_kernel gives VVH_KERNEL_DOT); q's
 * rows and k's rows must be whole heads (N % head_dim == 0), k and v alike,
 * head_dim a multiple of 16.  Like vvh_plan_set_input_op, the plan's device
 * table is rewritten in place after waiting for the device: set it before
 * capturing graphs that run the plan.  The plan keeps a device table of the
 * head_dim / 2 pair frequencies (1 / theta^(2i / head_dim), worked out once
 * by vvh_rope's arithmetic) until it is destroyed.  The position is an
 * argument of each run: vvh_plan_run_pos (vvh_plan_run runs at position 0). */
VVH_API int vvh_plan_set_rope(vvh_plan plan, size_t q_index, size_t k_index, size_t v_index, size_t head_dim,
                              float theta, void* k_cache, void* v_cache);
/* Cosine/sine table of a plan's RoPE epilogue (no reference counterpart):
 * the plan keeps cos and sin of every pair at positions [0, positions)
 * (positions * head_dim floats, worked out once by vvh_rope's arithmetic),
 * and runs whose rows all fall inside it read them instead of working them
 * out (the fp64 argument reduction of each pair); later positions still work
 * them out.  Changes no output bit.  Without it the table holds position 0
 * only.  positions in [1, 2^20]; the plan must have its RoPE epilogue.  Like
 * vvh_plan_set_rope it waits for the device and rewrites the plan's table in
 * place: call it before capturing graphs that run the plan.  The table
 * replaced stays allocated until the plan is destroyed (graphs captured
 * before may read it). */
VVH_API int vvh_plan_set_rope_table(vvh_plan plan, size_t positions);
/* SiLU-gated epilogue (no reference counterpart): problem `index` of the
 * plan has weights [gate | up] (N = 2 * inter rows, inter % 8 == 0, no
 * residual) and writes, instead of its N outputs per row, M rows of inter
 * values silu(gate) * up to its out: bit for bit what a plain run of the plan
 * followed by vvh_eltwise(VVH_OP_SILU_MUL) leaves there (each linear value
 * rounded to the output dtype, the product rounded once).  Saves the SiLU-mul
 * of a decode layer's MLP (transformer.h:180-183) from being repeated in
 * every block of the down projection's input stage.  The plan must run as one
 * k_dot_grouped launch (vvh_plan_kernel gives VVH_KERNEL_DOT).  Like
 * vvh_plan_set_input_op, the plan's device table is rewritten in place after
 * waiting for the device: set it before capturing graphs that run the plan. */
VVH_API int vvh_plan_set_glu(vvh_plan plan, size_t index);
/* vvh_plan_run with the position of activation row 0 for a RoPE epilogue. */
VVH_API int vvh_plan_run_pos(vvh_plan plan, size_t pos, void* stream);
/* Kernel family of a single-launch plan (VVH_KERNEL_DOT, VVH_KERNEL_STREAM
 * or VVH_KERNEL_SKINNY), or VVH_KERNEL_AUTO for a plan run as one launch per
 * problem. */
VVH_API int vvh_plan_kernel(vvh_plan plan, int* kernel);

/* ---- quantizer and data movement ----------------------------------------- */
/* Device restatement of quantize_per_channel (src/quantize/quantize.cc:9-48):
 * per row absmax -> scale = absmax/127 (IEEE division), codes =
 * clamp(round(w * (1/scale))) with ties away from zero, NaN -> 127; zero
 * rows get scale 0 and codes 0.  Codes and scales are bit-identical to the
 * host routine.  All pointers are device pointers. */
VVH_API int vvh_quantize_per_channel(const float* dev_weight, size_t N, size_t K,
                                     int8_t* dev_codes, float* dev_scales, void* stream);
/* Element type conversion on the device (f32<->f16, round to nearest even).
 * Replaces cuda_fp32_to_fp16 / cuda_fp16_to_fp32
 * (src/backend/cuda_kernels.h:69, :106). */
VVH_API int vvh_convert(void* dst, int dst_dtype, const void* src, int src_dtype, size_t n,
                        void* stream);
/* Fills n elements of dtype with mean + std * N(0,1) draws from a
 * counter-based generator (splitmix64 of seed and index, Box-Muller in fp32).
 * Deterministic for a given (seed, n); used to make synthetic weights and
 * activations resident in HBM without host traffic. */
VVH_API int vvh_fill_normal(void* dst, int dtype, size_t n, uint64_t seed, float mean, float std,
                            void* stream);

/* ---- dispatch introspection ---------------------------------------------- */
/* Kernel families of the linear path. */
/* ---- the other operators of a decode step ----------------------------------
 * Device restatements of the Backend operators transformer_forward
 * (include/vvllm/model/transformer.h:126-189) calls besides linear_q8, as
 * BackendCPU computes them (src/backend/backend_naive.cc; cited per entry).
 * Activations / outputs are device arrays of `dtype` (VVH_F32 or VVH_F16);
 * all arithmetic is fp32 with one rounding on store.  Weight-like inputs
 * (norm weights, biases, tables) are device fp32 arrays, e.g. from
 * vvh_mirror_f32.  Replaces BackendCUDA's versions
 * (src/backend/backend_cuda.cc:101-356) and their kernels. */
typedef enum vvh_op {
    VVH_OP_ADD = 0,       /* out = x + y          (backend_naive.cc:44-50) */
    VVH_OP_MUL = 1,       /* out = x * y          (:52-58) */
    VVH_OP_SILU = 2,      /* out = x / (1 + e^-x)  (:60-66) */
    VVH_OP_SILU_MUL = 3,  /* out = silu(x) * y    (:293-300) */
} vvh_op;
VVH_API int vvh_eltwise(int op, void* out, const void* x, const void* y, size_t n, int dtype, void* stream);
/* `rows` rows of RMSNorm: out = x / sqrt(mean(x^2) + eps) * weight (:68-76). */
VVH_API int vvh_rms_norm(void* out, const void* x, const float* dev_weight, size_t rows, size_t n, float eps,
                         int dtype, void* stream);
/* `rows` rows of softmax (:78-91). */
VVH_API int vvh_softmax(void* out, const void* x, size_t rows, size_t n, int dtype, void* stream);
/* Split-half RoPE in place on q [seq_len, num_heads, head_dim] and
 * k [seq_len, num_kv_heads, head_dim], positions pos.. (:93-137). */
VVH_API int vvh_rope(void* q, void* k, size_t seq_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
                     size_t pos, float theta, int dtype, void* stream);
/* vvh_rope, then the KV-cache append that follows it (transformer.h:145-160,
 * KVCache::append) in the same kernel: the rotated rows of k and the rows of
 * v [seq_len, num_kv_heads, head_dim] are also written to rows
 * pos .. pos + seq_len - 1 of k_cache and v_cache ([*, num_kv_heads,
 * head_dim], the caller's capacity).  No counterpart in the reference, which
 * copies the rows in separate calls; this saves the two copies per layer of
 * a decode step. */
VVH_API int vvh_rope_append(void* q, void* k, const void* v, void* k_cache, void* v_cache, size_t seq_len,
                            size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t pos, float theta, int dtype,
                            void* stream);
/* out[0..hidden) = table[token_id] (fp32 table [vocab, hidden]) (:338-342). */
VVH_API int vvh_embedding(void* out, const float* dev_table, size_t token_id, size_t hidden, size_t vocab, int dtype,
                          void* stream);
/* Causal attention for n_q consecutive queries (:344-378): query s of
 * q [n_q, num_heads, head_dim] attends to positions 0 .. len0 + s - 1 of
 * k, v [*, num_kv_heads, head_dim] (head h reads kv head
 * h / (num_heads / num_kv_heads)); out [n_q, num_heads * head_dim].  One call
 * replaces the model's per-query loop (transformer.h:168-173).  head_dim <= 256,
 * len0 + n_q - 1 <= 16000; a single query (n_q = 1, the decode step) with
 * head_dim a multiple of 8 up to 128, num_heads / num_kv_heads <= 16 and k, v
 * 16-byte aligned attends to up to 2^30 positions.  A single query over a
 * span long enough to split across blocks uses the stream's workspace; in
 * fp16 with head_dim 64 or 128 (and q 16-byte aligned) the blocks are merged
 * in the same launch through 64 KB of arrival counters per stream, allocated
 * by the stream's first such call: make that call before capturing graphs
 * on the stream, as for the workspace (vvh_workspace_release frees both). */
VVH_API int vvh_attention(void* out, const void* q, const void* k, const void* v, size_t n_q, size_t len0,
                          size_t num_heads, size_t num_kv_heads, size_t head_dim, float scale, int dtype,
                          void* stream);
/* Decode attention split for a merge in the next linear (no counterpart in the
 * reference: its transformer_forward runs attention and the o projection as
 * two calls, transformer.h:168-178).  For a single query (n_q = 1) in fp16,
 * head_dim 64 or 128, num_heads / num_kv_heads <= 16 and a span of at most
 * 512 positions, writes *nparts part rows per query head to parts: part p of
 * head h at parts + (p * num_heads + h) * (head_dim + 4), as head_dim
 * numerator floats, the running maximum (log2 units) and the exponential
 * sum.  parts_floats must cover *nparts * num_heads * (head_dim + 4) floats,
 * *nparts <= 8 (4 for spans of at most 256).  parts 16-byte aligned; other
 * shapes VVH_ERR_UNSUPPORTED.  vvh_linear_q8_dev_attn merges the parts into
 * exactly the fp16 row vvh_attention writes for the same call. */
VVH_API int vvh_attention_parts(float* parts, size_t parts_floats, size_t* nparts, const void* q, const void* k,
                                const void* v, size_t len0, size_t num_heads, size_t num_kv_heads,
                                size_t head_dim, float scale, int dtype, void* stream);
/* vvh_linear_q8_dev (M = 1, fp16 activations) of the attention row merged
 * from nparts parts of vvh_attention_parts (K = num_heads * head_dim): the
 * attention output and the o projection (+ residual, may alias out) of a
 * decode step in one launch, on the k_dot family, equal to vvh_attention
 * followed by vvh_linear_q8_dev on that family.  head_dim a power of two
 * dividing K (else VVH_ERR_INVALID_ARG); K % 16 == 0, K <= 1024, 16-byte
 * aligned parts and weights; otherwise VVH_ERR_UNSUPPORTED. */
VVH_API int vvh_linear_q8_dev_attn(void* out, const float* parts, size_t nparts, size_t head_dim,
                                   const int8_t* dev_weight, const float* dev_scales, const float* dev_bias,
                                   const void* residual, size_t N, size_t K, int out_dtype, void* stream);
/* Dense linear with fp32 or fp16 weights (wdtype): out[M,N] = x[M,K] . W[N,K]^T
 * + bias[N] (+ residual[M,N], may alias out) -- Backend::linear / linear_add
 * (:139-156, :302-320); the fp32 model path and the tied LM head. */
VVH_API int vvh_dense(void* out, const void* x, const void* dev_weight, int wdtype, const float* dev_bias,
                      const void* residual, size_t M, size_t N, size_t K, int dtype, void* stream);
/* out[M,N] = A[M,K] . B[K,N], B fp32 row-major (:25-42). */
VVH_API int vvh_matmul(void* out, const void* A, const float* dev_B, size_t M, size_t N, size_t K, int dtype,
                       void* stream);
/* Greedy sampling: *dev_index = the first index of the maximum of n fp32
 * logits, as std::max_element (src/sampler/sampler.cc:21-25). */
VVH_API int vvh_argmax(const float* logits, size_t n, int32_t* dev_index, void* stream);
/* Samples one index from n logits (dtype VVH_F32 or VVH_F16) into
 * *dev_index (device memory; nothing is copied to the host).  Replaces
 * cuda_sample (src/backend/cuda_kernels.h:107-111,
 * src/backend/cuda_kernels.cu:1322-1349) as SamplerCUDA::sample calls it
 * (src/sampler/sampler_cuda.cc:13-18), the reference's default decode
 * sampler (--temperature 0.7, bin/qwen/main.cc:29, :125-126).
 *   temperature == 0: vvh_argmax (the first index of the maximum).
 *   temperature  > 0: the Gumbel-max trick of sample_kernel (:1240-1317):
 *     argmax_i logit_i / temperature - log(-log(u_i)), with u_i the hash
 *     uniform of gpu_rand(seed, step, i) (:1228-1237), so a given (logits,
 *     temperature, seed, step) always gives the same index and successive
 *     steps draw independent samples of softmax(logit / temperature).  As
 *     there, only noisy values > -1e30 count (NaN never does) and the index
 *     is 0 if none does; equal noisy values resolve to the lower index.
 *   top_p is accepted and ignored, as cuda_sample does (:1325).
 * Unlike the reference (which exits the process on error and returns the
 * index through a blocking copy), a negative, NaN or infinite temperature is
 * VVH_ERR_INVALID_ARG and the call is asynchronous on `stream`. */
VVH_API int vvh_sample(const void* logits, int dtype, size_t n, float temperature, float top_p, uint64_t seed,
                       int32_t step, int32_t* dev_index, void* stream);
/* Device copy of a host fp32 array of n elements, as fp32 or converted to
 * fp16 (as_dtype), made on first use and kept (BackendCUDA::cache_weight /
 * cache_weight_as_fp16, backend_cuda.cc:51-95).  Keyed by (host, as_dtype):
 * the same host pointer with a different n is re-uploaded. */
VVH_API int vvh_mirror_f32(const float* host, size_t n, int as_dtype, const void** dev);
/* Drops the mirrors of a host array (both dtypes). */
VVH_API int vvh_mirror_release(const float* host);

typedef enum vvh_kernel {
    VVH_KERNEL_AUTO = 0,      /* size-based choice (default) */
    VVH_KERNEL_GENERIC = 1,   /* any shape / alignment, one thread per output */
    VVH_KERNEL_GEMV_F32 = 2,  /* fp32 activations, M < 16: VALU dot products */
    VVH_KERNEL_SKINNY = 3,    /* fp16 activations, M <= 64 (1, 2 or 4 groups of
                                 16 rows per weight chunk; plans: M <= 16),
                                 MFMA 16x16x32 */
    VVH_KERNEL_GEMM = 4,      /* LDS-tiled MFMA 32x32x16: fp16 activations, or
                                 fp32 activations (K % 64 == 0) split into
                                 fp16 high and low parts */
    VVH_KERNEL_STREAM = 5,    /* fp16 activations, M <= 16, K > 448: persistent
                                 streaming decode (large N, or grouped plans) */
    VVH_KERNEL_DOT = 6,       /* fp16 activations, M <= 16: weights loaded as
                                 whole cache lines of 8 rows; VALU dot products
                                 (M <= 2) or MFMA 16x16x32 (M >= 3) */
} vvh_kernel;
/* Which kernel family vvh_linear_q8 would use for this call (after the
 * override below); returns a vvh_kernel value, or a negative status. */
VVH_API int vvh_linear_q8_choice(size_t M, size_t N, size_t K, int act_dtype, int out_dtype);
/* The GEMM kernel behind VVH_KERNEL_GEMM for an fp16 call of this shape
 * (measurement and reporting; no reference counterpart): returns 3 for
 * k_gemm3 on 128-row tiles, 4 for k_gemm3 on 64-row tiles (*tile_n = 128
 * or 192), 1 for k_gemm (K % 64 != 0), or a negative status; *splits > 1 is
 * a split-K launch followed by a reduction kernel.  tile_n and splits may
 * be NULL. */
VVH_API int vvh_gemm_variant(size_t M, size_t N, size_t K, int* tile_n, int* splits);
/* Forces one kernel family for subsequent calls on this process (testing and
 * measurement); VVH_KERNEL_AUTO restores the size-based choice.  A forced
 * family that cannot serve a call falls back to GENERIC. */
VVH_API int vvh_set_kernel_override(int kernel);

#ifdef __cplusplus
}
#endif

#endif /* VVLLM_HIP_H */
