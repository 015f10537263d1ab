"""CPU-side tests of the C ABI (no GPU needed, no compute calls).

* libvvllm_hip.so loads and exports every VVH_API function that
  include/vvllm_hip.h declares, and the ctypes table binds exactly those;
* argument validation happens on the host and returns status codes (the
  reference's linear_q8 path checks no arguments);
* the kernel-family choice of the dispatcher;
* the caching allocator logic (tests/cpp/test_pool.cc, with a fake backing
  allocator, built with ASan/UBSan);
* libvvllm_backend_hip.so (BackendHIP) links and loads.
"""
import ctypes
import os
import re
import subprocess

import pytest

from vvllm_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vvllm_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return re.findall(r"VVH_API\s+[\w\s\*]+?\b(vvh_\w+)\s*\(", text)


def test_header_declares_and_library_exports_every_symbol():
    lib = capi.load()
    names = declared_functions()
    assert len(names) >= 30
    for n in names:
        assert hasattr(lib, n), f"{n} declared in vvllm_hip.h but not exported"
    assert set(names) == set(capi.SIGNATURES), "ctypes table out of sync with the header"


def test_only_the_c_abi_is_exported():
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == set(declared_functions())


def test_status_strings_and_version():
    lib = capi.load()
    for code, name in capi.STATUS.items():
        assert lib.vvh_status_string(code).decode() == name
    assert lib.vvh_status_string(99).decode() == "VVH_ERR_UNKNOWN_STATUS"
    assert b"gfx950" in lib.vvh_version()


def test_validation_before_device_use():
    st = capi.status_of
    P = 0x1000  # never dereferenced: every call below fails validation first
    # bad dtypes
    assert st("vvh_linear_q8_dev", P, P, P, P, None, None, 1, 16, 16, 7, 0, None) == 1
    assert st("vvh_linear_q8_dev", P, P, P, P, None, None, 1, 16, 16, 0, -1, None) == 1
    # null out / scales / weight
    assert st("vvh_linear_q8_dev", None, P, P, P, None, None, 1, 16, 16, 0, 0, None) == 1
    assert st("vvh_linear_q8_dev", P, P, P, None, None, None, 1, 16, 16, 0, 0, None) == 1
    assert st("vvh_linear_q8_dev", P, P, None, P, None, None, 1, 16, 16, 1, 0, None) == 1
    assert "null" in capi.load().vvh_last_error().decode()
    # size overflow
    assert st("vvh_linear_q8_dev", P, P, P, P, None, None, 1 << 40, 1 << 40, 16, 0, 0, None) == 1
    # empty problems are no-ops, even before init
    assert st("vvh_linear_q8_dev", None, None, None, None, None, None, 0, 16, 16, 0, 0, None) == 0
    assert st("vvh_linear_q8_dev", None, None, None, None, None, None, 4, 0, 16, 0, 0, None) == 0
    # valid arguments but no vvh_init in this process -> NOT_INITIALIZED, not a crash
    assert st("vvh_linear_q8_dev", P, P, P, P, None, None, 1, 16, 16, 0, 0, None) == 5
    assert st("vvh_sync") == 5
    # weight registry / plans: argument checks
    h = ctypes.c_uint64(7)
    assert st("vvh_weight_register", None, P, None, 4, 4, ctypes.byref(h)) == 1 and h.value == 0
    assert st("vvh_weight_register", P, P, None, 0, 4, ctypes.byref(h)) == 1
    assert st("vvh_weight_register", P, P, None, 4, 4, None) == 1
    assert st("vvh_weight_find", P, ctypes.byref(h)) == 6
    assert st("vvh_weight_release", 12345) == 6
    assert st("vvh_plan_run", 999, None) == 5
    assert st("vvh_plan_destroy", 999) == 6
    plan = ctypes.c_uint64()
    assert st("vvh_plan_create", None, 0, 1, 1, ctypes.byref(plan)) == 1
    probs = (capi.Q8Problem * 1)()
    probs[0].M, probs[0].N, probs[0].K = 1, 16, 16  # null pointers
    assert st("vvh_plan_create", probs, 1, 1, 1, ctypes.byref(plan)) == 1
    assert st("vvh_convert", P, 3, P, 0, 10, None) == 1
    assert st("vvh_fill_normal", None, 0, 10, 1, 0.0, 1.0, None) == 1
    assert st("vvh_quantize_per_channel", None, 4, 4, P, P, None) == 1
    assert st("vvh_set_kernel_override", 9) == 1
    # weight ingestion: source dtype must be F32 or BF16, pointers and shape valid
    sc = (ctypes.c_float * 4)()
    assert st("vvh_weight_ingest", P, capi.F16, None, 4, 4, sc, ctypes.byref(h)) == 1
    assert st("vvh_weight_ingest", None, capi.BF16, None, 4, 4, sc, ctypes.byref(h)) == 1
    assert st("vvh_weight_ingest", P, capi.BF16, None, 4, 4, None, ctypes.byref(h)) == 1
    assert st("vvh_weight_ingest", P, capi.BF16, None, 0, 4, sc, ctypes.byref(h)) == 1
    assert st("vvh_weight_ingest", P, capi.BF16, None, 1 << 40, 1 << 40, sc, ctypes.byref(h)) == 1
    assert st("vvh_weight_ingest", P, capi.BF16, None, 4, 4, sc, None) == 1
    assert st("vvh_weight_ingest", P, capi.BF16, None, 4, 4, sc, ctypes.byref(h)) == 5  # before vvh_init
    # input stages of a decode linear: refused shapes and arguments, before any device use
    def lin_in(M, K, act, op, w):
        return st("vvh_linear_q8_dev_in", P, P, P, P, None, None, M, 16, K, act, act, op, w, 1e-6, None)
    assert lin_in(1, 896, capi.F16, 3, P) == 1                    # unknown stage
    assert lin_in(1, 896, capi.F16, capi.IN_RMS_NORM, None) == 1  # RMSNorm without weights
    assert lin_in(1, 896, capi.F16, capi.IN_RMS_NORM, P + 4) == 1  # misaligned weights
    assert lin_in(5, 896, capi.F16, capi.IN_RMS_NORM, P) == 7     # M > 4
    assert lin_in(1, 896, capi.F32, capi.IN_SILU_MUL, None) == 7  # fp32 activations
    assert lin_in(1, 888, capi.F16, capi.IN_SILU_MUL, None) == 7  # K % 16 != 0
    assert lin_in(4, 20000, capi.F16, capi.IN_SILU_MUL, None) == 7  # rows beyond the LDS
    assert lin_in(1, 896, capi.F16, capi.IN_RMS_NORM, P) == 5     # valid, before vvh_init
    assert lin_in(1, 896, capi.F16, capi.IN_NONE, None) == 5      # no stage: vvh_linear_q8_dev
    # RoPE + KV append
    assert st("vvh_rope_append", P, P, P, P, P, 1, 14, 2, 63, 0, 1e4, capi.F16, None) == 1  # odd head_dim
    assert st("vvh_rope_append", P, P, P, None, P, 1, 14, 2, 64, 0, 1e4, capi.F16, None) == 1  # no key cache
    assert st("vvh_rope_append", P, P, P, P, P, 1, 14, 2, 64, 0, 1e4, 9, None) == 1  # bad dtype
    assert st("vvh_rope_append", P, P, P, P, P, 1, 14, 2, 64, 0, 1e4, capi.F16, None) == 5
    assert st("vvh_plan_set_input_op", 999, capi.IN_RMS_NORM, P, 1e-6) == 5
    # sampler: temperature must be finite and >= 0, logits F32 / F16, n >= 1
    for T in (-0.5, float("nan"), float("inf")):
        assert st("vvh_sample", P, capi.F32, 16, T, 1.0, 1, 0, P, None) == 1
    assert st("vvh_sample", P, 5, 16, 1.0, 1.0, 1, 0, P, None) == 1
    assert st("vvh_sample", P, capi.F32, 0, 1.0, 1.0, 1, 0, P, None) == 1
    assert st("vvh_sample", None, capi.F32, 16, 1.0, 1.0, 1, 0, P, None) == 1
    assert st("vvh_sample", P, capi.F32, 16, 0.7, 0.9, 1, 0, None, None) == 1
    assert st("vvh_sample", P, capi.F16, 16, 0.7, 0.9, 1, 0, P, None) == 5
    stats = capi.PoolStats()
    assert st("vvh_pool_get_stats", ctypes.byref(stats)) == 0 and stats.bytes_in_use == 0


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_init_without_device_reports_no_device():
    buf = ctypes.create_string_buffer(64)
    assert capi.status_of("vvh_init", 0, buf, 64) == 2
    assert capi.load().vvh_device_cu_count() == 0


def test_gemm_variant_choice():
    """The GEMM kernel behind the "gemm" family (host logic, 256 CUs assumed
    off the device): k_gemm3 with 64 x 128 tiles when those give each block
    a CU, 128 x 128 tiles when one round of blocks covers the problem,
    128 x 192 when that saves a round, split-K (on 64 x 128 tiles) for few
    tiles over a long K, k_gemm for K % 64 != 0."""
    assert capi.gemm_variant(512, 4864, 896) == "k_gemm3 128x128"     # 304 64-row tiles; 152, one round
    assert capi.gemm_variant(128, 4864, 896) == "k_gemm3 64x64"       # 152 64 x 64 tiles, one round
    assert capi.gemm_variant(512, 1152, 896) == "k_gemm3 64x64"       # 144
    assert capi.gemm_variant(256, 4864, 512) == "k_gemm3 64x128"      # 304 64 x 64 tiles, 152 64 x 128
    assert capi.gemm_variant(256, 8960, 1536) == "k_gemm3 128x128"    # 280 64-row tiles > 256 CUs
    assert capi.gemm_variant(2048, 4864, 896) == "k_gemm3 128x192"    # 3 rounds -> 2
    assert capi.gemm_variant(512, 896, 4864) == "k_gemm3 64x128 split 4"    # 56 64-row tiles, 76 k stages
    assert capi.gemm_variant(2048, 896, 4864) == "k_gemm3 64x128"   # 224 64-row tiles beat 2 splits
    assert capi.gemm_variant(64, 1536, 1536) == "k_gemm3 64x64 split 4"     # 24 tiles, 24 k stages
    assert capi.gemm_variant(128, 896, 4864) == "k_gemm3 64x64 split 7"     # 28 tiles, 76 k stages
    assert capi.gemm_variant(256, 1536, 8960) == "k_gemm3 64x128 split 5"   # 64 x 64 would halve the count
    assert capi.gemm_variant(256, 1536, 1536) == "k_gemm3 64x64"    # 96 64 x 64 tiles beat splits
    assert capi.gemm_variant(300, 1000, 80) == "k_gemm"               # K % 64 != 0
    assert capi.load().vvh_gemm_variant(0, 16, 64, None, None) == -1  # -VVH_ERR_INVALID_ARG


def test_dispatch_choice():
    ch = capi.kernel_choice
    try:
        capi.set_kernel(capi.KERNEL_AUTO)
        assert ch(1, 896, 896, capi.F32, capi.F32) == "gemv_f32"      # config 1
        assert ch(15, 4864, 896, capi.F32, capi.F32) == "gemv_f32"
        assert ch(16, 4864, 896, capi.F32, capi.F32) == "gemm"        # fp32 prefill on MFMA
        assert ch(512, 4864, 880, capi.F32, capi.F32) == "gemv_f32"   # K % 64 != 0
        assert ch(1, 151936, 896, capi.F16, capi.F32) == "dot"        # config 3 (M = 1)
        assert ch(1, 896, 896, capi.F16, capi.F16) == "dot"           # config 2 (M = 1)
        assert ch(2, 896, 896, capi.F16, capi.F16) == "dot"           # M = 2
        assert ch(2, 151936, 896, capi.F16, capi.F32) == "dot"        # M = 2, 9496 tiles
        assert ch(4, 896, 896, capi.F16, capi.F16) == "dot"           # M = 3, 4 on few tiles
        assert ch(4, 1536, 8960, capi.F16, capi.F16) == "dot"
        assert ch(3, 9728, 896, capi.F16, capi.F16) == "dot"          # M = 3, 608 tiles
        assert ch(3, 17920, 1536, capi.F16, capi.F16) == "dot"        # M = 3, 1120 tiles: the activation tile
        assert ch(5, 1536, 8960, capi.F16, capi.F16) == "dot"         # M = 5..8 below 1024 tiles
        assert ch(8, 896, 4864, capi.F16, capi.F16) == "dot"
        assert ch(8, 4864, 896, capi.F16, capi.F16) == "dot"
        assert ch(5, 17920, 1536, capi.F16, capi.F16) == "dot"        # >= 1024 tiles, early launch re-reading
        assert ch(8, 17920, 1536, capi.F16, capi.F16) == "dot"        #   >= 5 MB of activations, <= 12 k steps
        assert ch(8, 151936, 896, capi.F16, capi.F16) == "dot"        #   per wave
        assert ch(16, 151936, 896, capi.F16, capi.F16) == "dot"
        assert ch(16, 200000, 896, capi.F16, capi.F16) == "gemm"      # not an early launch: no activation tile
        assert ch(4, 65536, 4096, capi.F16, capi.F16) == "skinny"     # 32 k steps per wave: no activation tile
        assert ch(9, 1536, 8960, capi.F16, capi.F16) == "dot"         # long rows, few tiles, M <= 10
        assert ch(10, 1536, 8960, capi.F16, capi.F16) == "dot"
        assert ch(11, 1536, 8960, capi.F16, capi.F16) == "gemm"
        assert ch(12, 896, 4864, capi.F16, capi.F16) == "dot"
        assert ch(16, 896, 4864, capi.F16, capi.F16) == "dot"         # M * K <= 16 * 4864
        assert ch(13, 1536, 8960, capi.F16, capi.F16) == "gemm"       # long rows, few tiles: split-K GEMM
        assert ch(9, 8960, 1536, capi.F16, capi.F16) == "dot"         # M > 8 below 1024 tiles, short rows
        assert ch(16, 17920, 1536, capi.F16, capi.F16) == "dot"       # M > 8 on 1120 tiles (activation tile)
        assert ch(16, 4096, 8192, capi.F16, capi.F16) == "gemm"       # M > 8, long rows on 256 tiles
        assert ch(5, 151936, 896, capi.F16, capi.F32) == "dot"        # streaming only when forced
        assert ch(16, 4864, 896, capi.F16, capi.F16) == "dot"         # M > 8 on 304 tiles
        assert ch(16, 1536, 8960, capi.F16, capi.F16) == "gemm"       # M > 10 on long rows
        assert ch(16, 1536, 1536, capi.F16, capi.F16) == "dot"        # M > 8, few tiles, short rows
        assert ch(17, 4864, 896, capi.F16, capi.F16) == "gemm"        # M > 16 on 304 tiles
        assert ch(17, 1152, 896, capi.F16, capi.F16) == "skinny"      # M > 16: 2-4 groups of 16 rows
        assert ch(64, 896, 896, capi.F16, capi.F16) == "skinny"       #   on few tiles, M * K <= 64 * 896
        assert ch(32, 1536, 1536, capi.F16, capi.F16) == "skinny"
        assert ch(48, 1536, 1536, capi.F16, capi.F16) == "gemm"
        assert ch(32, 896, 4864, capi.F16, capi.F16) == "gemm"
        assert ch(65, 896, 896, capi.F16, capi.F16) == "gemm"
        assert ch(512, 4864, 896, capi.F16, capi.F16) == "gemm"       # config 4
        assert ch(1, 2, 2, capi.F32, capi.F32) == "generic"           # K % 16 != 0
        assert ch(4, 16, 0, capi.F16, capi.F16) == "generic"          # K == 0
        capi.set_kernel(capi.KERNEL_GEMM)
        assert ch(1, 896, 896, capi.F16, capi.F16) == "gemm"
        assert ch(1, 896, 896, capi.F32, capi.F32) == "gemm"          # fp32 split into fp16 hi/lo
        assert ch(40, 896, 880, capi.F32, capi.F32) == "generic"      # fp32 needs K % 64 == 0
        capi.set_kernel(capi.KERNEL_SKINNY)
        assert ch(64, 896, 896, capi.F16, capi.F16) == "skinny"
        assert ch(65, 896, 896, capi.F16, capi.F16) == "generic"      # M > 64
        capi.set_kernel(capi.KERNEL_DOT)
        assert ch(1, 16, 16, capi.F16, capi.F16) == "dot"
        assert ch(16, 16, 16, capi.F16, capi.F16) == "dot"
        assert ch(17, 16, 16, capi.F16, capi.F16) == "generic"        # M > 16
        assert ch(1, 16, 16, capi.F32, capi.F32) == "generic"         # fp32 activations
        capi.set_kernel(capi.KERNEL_STREAM)
        assert ch(1, 16, 512, capi.F16, capi.F16) == "stream"
        assert ch(1, 16, 448, capi.F16, capi.F16) == "generic"        # fewer than 8 k steps
        assert ch(17, 896, 896, capi.F16, capi.F16) == "generic"      # M > 16
    finally:
        capi.set_kernel(capi.KERNEL_AUTO)


def test_pool_logic_binary():
    exe = os.path.join(ROOT, "tests", "cpp", "bin", "test_pool")
    if not os.path.exists(exe):
        from vvllm_amd import build
        build.build_test_pool()
    p = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert p.returncode == 0, p.stdout + p.stderr


def test_backend_library_links():
    path = os.path.join(ROOT, "vvllm_amd", "lib", "libvvllm_backend_hip.so")
    assert os.path.exists(path)
    ctypes.CDLL(path)  # resolves libvvllm_hip.so through its rpath
    out = subprocess.run(["nm", "-DC", "--defined-only", path], capture_output=True, text=True).stdout
    for sym in ("vvllm::BackendHIP::linear_q8(", "vvllm::BackendHIP::linear_q8_add(",
                "vvllm::hip_device_allocate("):
        assert sym in out
