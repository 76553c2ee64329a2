"""The C-ABI library: it loads, exports what include/nibblegemm_amd.h declares,
and rejects every argument the reference's host checks reject -- all before
any HIP call, so this runs on a machine without a GPU.

The pointer values passed here are never dereferenced: every call either
fails validation (which happens before any HIP call) or is the M > 8 case that
the launcher refuses before touching the device.
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nibblegemm_amd.h")

OK, INVALID, UNSUPPORTED, WORKSPACE, HIP = 0, 1, 2, 3, 4
P = 1 << 20  # aligned, never dereferenced


def declared_functions():
    text = open(HEADER).read()
    return re.findall(r"NIBBLE_API\s+[\w\s\*]+?\b(nibble_\w+)\s*\(", text)


def test_header_declares_the_entry_points():
    names = set(declared_functions())
    assert {"nibble_abi_version", "nibble_last_error", "nibble_gemv_w4a16",
            "nibble_gemv_workspace_bytes", "nibble_gemv_counter_bytes", "nibble_gemm_w4a16",
            "nibble_gemm_workspace_bytes", "nibble_gemm_counter_bytes",
            "nibble_dequant_w4"} <= names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_native.LIBRARY_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
    lib.nibble_abi_version.restype = ctypes.c_int
    version = int(re.search(r"#define NIBBLE_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.nibble_abi_version() == version


def test_binding_loads_and_matches_abi():
    ext = ng.extension()
    assert ext.abi_version() == _native.ABI_VERSION


def gemv(ext, M, K, N, g=128, wq_rows=None, s_rows=None, s_cols=None, version=4, splits=0,
         threads=0, ptr=P):
    wq_rows = K // 8 if wq_rows is None else wq_rows
    s_rows = (K // g if g else 0) if s_rows is None else s_rows
    s_cols = N if s_cols is None else s_cols
    return ext.gemv(ptr, M, K, ptr, wq_rows, N, ptr, s_rows, s_cols, g, version, splits, threads,
                    ptr, None, 0, None)


@pytest.mark.parametrize("kwargs,needle", [
    (dict(M=1, K=256, N=128, wq_rows=31), "packed weight rows"),
    (dict(M=1, K=256, N=128, s_rows=3), "scale rows"),
    (dict(M=1, K=256, N=128, s_cols=132), "scale columns"),
    (dict(M=1, K=256, N=130), "multiple of 4"),
    (dict(M=1, K=256, N=128, g=32, s_rows=8), "group_size"),
    (dict(M=1, K=256, N=128, version=5), "version"),
    (dict(M=1, K=256, N=128, ptr=P + 2), "misaligned"),
    (dict(M=1, K=256, N=128, ptr=0), "null"),
])
def test_gemv_rejections(kwargs, needle):
    ext = ng.extension()
    rc = gemv(ext, **kwargs)
    assert rc == INVALID
    assert needle in ext.last_error()


@pytest.mark.parametrize("version", [3, 4])
def test_gemv_rejects_m_above_8(version):
    ext = ng.extension()
    assert gemv(ext, 9, 256, 132, version=version) == UNSUPPORTED
    assert "M <= 8" in ext.last_error()


def test_gemv_threads_override_validated():
    ext = ng.extension()
    assert gemv(ext, 1, 256, 128, threads=96) == INVALID
    assert "block_threads" in ext.last_error()
    # the reference's 32-thread block is accepted and planned as one wave
    assert ext.gemv_workspace_bytes(1, 1024, 256, 64, 4, 16, 32, None) == \
        ext.gemv_workspace_bytes(1, 1024, 256, 64, 4, 16, 64, None)


def test_gemm_workspace_formula():
    """Batches of M <= 32 run the streaming kernels (split-K workspace as for
    gemv), as do M <= 64 whose one 64-row block fills the CUs in one round
    and M <= 128 whose passes over the weights (one per 32 rows) stay under
    48 MiB; otherwise tiles, split over K only when the tiles are few."""
    ext = ng.extension()
    assert ext.gemm_workspace_bytes(16, 14336, 4096, 128, 6, None) == (256 + 4 * 16 * 4096 * 4, 256)
    assert ext.gemm_workspace_bytes(32, 4096, 14336, 128, 7, None) == (0, 0)
    # M = 33..64 over 29.4 MB of weights: one 64-row block of the batch
    # kernel, 64 strips split 4 ways (256 workgroups), both versions
    assert ext.gemm_workspace_bytes(33, 14336, 4096, 128, 6, None) == (256 + 4 * 33 * 4096 * 4, 256)
    assert ext.gemm_workspace_bytes(33, 14336, 4096, 128, 7, None) == (256 + 4 * 33 * 4096 * 4, 256)
    # 4096 x 14336: 224 strips unsplit at M = 64 (one block), 224 unsplit
    # 64-row tiles at M = 128
    assert ext.gemm_workspace_bytes(64, 4096, 14336, 128, 6, None) == (0, 0)
    assert ext.gemm_workspace_bytes(128, 4096, 14336, 128, 6, None) == (0, 0)
    # 4096 x 4096: one 64-row block at M = 33, its 64 strips split 4 ways;
    # 4096 x 6144 (192 workgroups at most) streams 32-row blocks, unsplit
    assert ext.gemm_workspace_bytes(33, 4096, 4096, 128, 6, None) == (256 + 4 * 33 * 4096 * 4, 256)
    assert ext.gemm_workspace_bytes(33, 4096, 6144, 128, 6, None) == (0, 0)
    # M > 128 runs the producer/consumer kernel; over a long K (224 steps of
    # 64) with 128 x 128 tiles split by their count: 2 x 32 = 64 tiles 4 ways
    # (both versions: the same plan, so the same bits)
    assert ext.gemm_workspace_bytes(129, 14336, 4096, 128, 6, None) == (256 + 4 * 129 * 4096 * 4, 256)
    assert ext.gemm_workspace_bytes(129, 14336, 4096, 128, 7, None) == (256 + 4 * 129 * 4096 * 4, 256)
    # 3 x 32 = 96 and 4 x 32 = 128 tiles split 2 ways; 1536 rows (384 tiles,
    # a round and a half of the CUs) 2 ways; counters padded to 512 bytes
    assert ext.gemm_workspace_bytes(384, 14336, 4096, 128, 6, None) == (512 + 2 * 384 * 4096 * 4, 512)
    assert ext.gemm_workspace_bytes(512, 14336, 4096, 128, 6, None) == (512 + 2 * 512 * 4096 * 4, 512)
    assert ext.gemm_workspace_bytes(1536, 14336, 4096, 128, 6, None) == \
        (1536 + 2 * 1536 * 4096 * 4, 1536)
    # 4096 <= K < 8192 with few 64-row tiles: 4 ways (4096 x 4096, M = 129:
    # 3 x 32 = 96 tiles); 4096 x 6144 at M = 256 (192 tiles) runs unsplit,
    # as does version 7 (128-row tiles)
    assert ext.gemm_workspace_bytes(129, 4096, 4096, 128, 6, None) == (512 + 4 * 129 * 4096 * 4, 512)
    assert ext.gemm_workspace_bytes(256, 4096, 6144, 128, 6, None) == (0, 0)
    assert ext.gemm_workspace_bytes(129, 4096, 4096, 128, 7, None) == (0, 0)
    # N % 4 != 0 cannot stream nor take 16-byte B loads: the tile kernel, 33
    # tiles of 64 x 128, split 4 ways
    assert ext.gemm_workspace_bytes(16, 14336, 4098, 128, 6, None) == (256 + 4 * 16 * 4098 * 4, 256)
    # 192 and 256 tiles of 128 x 128 are not split; above 128 rows a short K
    # never splits
    assert ext.gemm_workspace_bytes(768, 14336, 4096, 128, 6, None) == (0, 0)
    assert ext.gemm_workspace_bytes(1024, 14336, 4096, 128, 7, None) == (0, 0)
    assert ext.gemm_workspace_bytes(512, 4096, 14336, 128, 6, None) == (0, 0)
    # from M = 1024 version 6 takes 256 x 256 tiles where they make one round
    # of the CUs (224 tiles here), never split; from M = 2048, 256 x 128
    # tiles where they make whole rounds (256 at 2048 x 4096), never split
    assert ext.gemm_workspace_bytes(1024, 4096, 14336, 128, 6, None) == (0, 0)
    assert ext.gemm_workspace_bytes(2048, 14336, 4096, 128, 6, None) == (0, 0)
    # 3072 x 4096: 384 such tiles, a round and a half, so 128 x 128 tiles
    # (768, enough not to split)
    assert ext.gemm_workspace_bytes(3072, 14336, 4096, 128, 6, None) == (0, 0)
    # version 7 keeps 128 x 128 tiles: 16 x 32 of them at M = 2048, no split
    assert ext.gemm_workspace_bytes(2048, 14336, 4096, 128, 7, None) == (0, 0)
    assert ext.gemm_workspace_bytes(16, 14336, 4096, 128, 5, None) == (0, 0)


def test_gemv_workspace_formula():
    ext = ng.extension()
    # 1024 / 64 = 16 groups split 16 ways over four 64-column strips:
    # 256 bytes of counters (padded), then 16 x M x N fp32 partials.
    ws, counters = ext.gemv_workspace_bytes(1, 1024, 256, 64, 4, 16, 0, None)
    assert counters == 256
    assert ws == 256 + 16 * 1 * 256 * 4
    # floor-then-trim: 32 groups asked for 27 splits -> 1 group each -> 32 splits
    ws, counters = ext.gemv_workspace_bytes(2, 4096, 512, 128, 4, 27, 0, None)
    assert counters == 256 and ws == 256 + 32 * 2 * 512 * 4
    # a single split needs no workspace
    assert ext.gemv_workspace_bytes(1, 1024, 256, 64, 4, 1, 0, None) == (0, 0)
    assert ext.gemv_workspace_bytes(1, 1024, 256, 64, 3, 0, 0, None) == (0, 0)
    # default plan at the benchmark decode shapes (pure host arithmetic): the
    # strip kernel (no workspace) up to K = 8192; beyond, the split kernel
    # with ~8 groups per wave of 4
    assert ext.gemv_workspace_bytes(1, 4096, 14336, 128, 4, 0, 0, None) == (0, 0)
    assert ext.gemv_workspace_bytes(1, 4096, 4096, 128, 4, 0, 0, None) == (0, 0)
    assert ext.gemv_workspace_bytes(1, 8192, 8192, 128, 4, 0, 0, None) == (0, 0)
    assert ext.gemv_workspace_bytes(1, 14336, 4096, 128, 4, 0, 0, None) == (256 + 4 * 4096 * 4, 256)
    # an explicit split count always runs the split kernel
    assert ext.gemv_workspace_bytes(1, 8192, 8192, 128, 4, 2, 0, None) == (512 + 2 * 8192 * 4, 512)
    # 14336 / 64 = 224 strips of counters need 896 bytes, padded to 1024
    assert ext.gemv_workspace_bytes(2, 16384, 14336, 128, 4, 0, 0, None) == (
        1024 + 4 * 2 * 14336 * 4, 1024)
    # invalid requests report zero
    assert ext.gemv_workspace_bytes(9, 1024, 256, 64, 4, 4, 0, None) == (0, 0)
    assert ext.gemv_workspace_bytes(1, 1024, 256, 32, 4, 4, 0, None) == (0, 0)


def gemm(ext, M, K, N, g=128, wq_rows=None, s_rows=None, s_cols=None, version=6, ptr=P):
    wq_rows = K // 8 if wq_rows is None else wq_rows
    s_rows = K // g if s_rows is None else s_rows
    s_cols = N if s_cols is None else s_cols
    return ext.gemm(ptr, M, K, ptr, wq_rows, N, ptr, s_rows, s_cols, g, version, ptr, None, 0,
                    None)


@pytest.mark.parametrize("kwargs,needle", [
    (dict(M=16, K=256, N=128, wq_rows=31), "packed weight rows"),
    (dict(M=16, K=264, N=128, g=8, s_rows=33), "multiple of 32"),
    (dict(M=16, K=256, N=127), "even"),
    (dict(M=16, K=256, N=128, g=32, s_rows=8), "group_size"),
    (dict(M=16, K=256, N=128, s_rows=1), "scale rows"),
    (dict(M=16, K=256, N=128, s_cols=130), "scale columns"),
    (dict(M=16, K=256, N=128, version=5), "version"),
    (dict(M=1 << 20, K=4096, N=1024), "32-bit indexing"),
    (dict(M=16, K=256, N=128, ptr=P + 8), "misaligned"),
])
def test_gemm_rejections(kwargs, needle):
    ext = ng.extension()
    assert gemm(ext, **kwargs) == INVALID
    assert needle in ext.last_error()


@pytest.mark.parametrize("args,needle", [
    ((P, 32, 128, P, 3, 128, 128), "scale rows"),
    ((P, 32, 128, P, 2, 132, 128), "scale columns"),
    ((P, 32, 128, P, 2, 128, 100), "group_size"),
    ((P, 32, 128, P, 1, 128, 192), "divisible"),
    ((0, 32, 128, P, 2, 128, 128), "null"),
])
def test_dequant_rejections(args, needle):
    ext = ng.extension()
    wq, rows, n, s, sr, sc, g = args
    assert ext.dequant(wq, rows, n, s, sr, sc, g, 1, P, None) == INVALID
    assert needle in ext.last_error()


def test_noalloc_gemv_rejects_plans_beyond_its_scratch():
    """nibble_gemv_w4a16_noalloc refuses, before any HIP call, a split plan
    whose partials exceed its static scratch (4 MiB less 64 KiB of counters),
    with a message that names the limit; validation errors are
    nibble_gemv_w4a16's."""
    lib = ctypes.CDLL(_native.LIBRARY_PATH)
    fn = lib.nibble_gemv_w4a16_noalloc
    fn.restype = ctypes.c_int
    fn.argtypes = ([ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64] * 3
                   + [ctypes.c_int64] * 4 + [ctypes.c_void_p, ctypes.c_void_p])
    lib.nibble_last_error.restype = ctypes.c_char_p
    # 16 splits x 8 rows x 8192 columns of fp32 partials = 4 MiB
    rc = fn(P, 8, 4096, P, 512, 8192, P, 32, 8192, 128, 4, 16, 0, P, None)
    assert rc == 2 and b"static scratch" in lib.nibble_last_error()
    # (a plan that fits would launch, which needs a GPU: tests/test_zz_no_alloc.py)
    rc = fn(P, 9, 4096, P, 512, 8192, P, 32, 8192, 128, 4, 0, 0, P, None)
    assert rc == 2 and b"M <= 8" in lib.nibble_last_error()
    rc = fn(P, 1, 4096, P, 511, 8192, P, 32, 8192, 128, 4, 0, 0, P, None)
    assert rc == INVALID and b"packed weight rows" in lib.nibble_last_error()


def test_gemv_timeline_setter_checks_its_buffer():
    """nibble_gemv_timeline (diagnostics) is host state only: it rejects a
    misaligned or empty buffer and NULL turns it off; no device call."""
    ext = ng.extension()
    try:
        assert ext.gemv_timeline(P + 4, 4096) == INVALID
        assert "alignment" in ext.last_error()
        assert ext.gemv_timeline(P, 0) == INVALID
        assert "positive size" in ext.last_error()
        assert ext.gemv_timeline(P, 4096) == OK
    finally:
        assert ext.gemv_timeline(None, 0) == OK


def test_binding_rejects_wrong_arity():
    ext = ng.extension()
    with pytest.raises(TypeError):
        ext.gemv(1, 2, 3)


# --------------------------------------------------------------------------
# Python layer: errors raised before any device work
# --------------------------------------------------------------------------
def _cpu_case(M=1, K=256, N=128, g=128):
    qw = ng.quantize(torch.randn(K, N) * 0.02, group_size=g)
    X = torch.randn(M, K).half()
    return X, qw


def test_matmul_rejects_k_mismatch_and_rank():
    X, qw = _cpu_case()
    with pytest.raises(ValueError):
        ng.matmul(torch.randn(1, 128).half(), qw)
    with pytest.raises(ValueError):
        ng.matmul(X.reshape(1, 1, 256), qw)


def test_kernels_refuse_host_tensors():
    X, qw = _cpu_case()
    with pytest.raises(RuntimeError, match="GPU"):
        ng.gemv(X, qw)
    with pytest.raises(RuntimeError, match="GPU"):
        ng.gemm(X, qw)
    with pytest.raises(RuntimeError, match="GPU"):
        ng.dequant(qw)


def test_library_loads_only_one_hip_runtime():
    """The library resolves libamdhip64 to the runtime torch already loaded."""
    ng.extension()
    maps = [l for l in open("/proc/self/maps") if "libamdhip64" in l]
    paths = {l.split()[-1] for l in maps}
    assert len(paths) <= 1, paths


REFERENCE_NAMES = ("DECODE_MAX_M", "QuantLinear", "QuantizedWeight", "dequant", "dequantize",
                   "HessianAccumulator", "extension", "find_decoder_blocks", "gptq_quantize",
                   "quantize_model_gptq", "gemm", "gemv", "matmul", "pack_nibbles", "quantize",
                   "reference_matmul", "unpack_nibbles")


def test_package_keeps_the_reference_namespace():
    """Every name the reference package exports (python/nibblegemm/__init__.py:
    19-37) is exported here; the offline GPTQ quantiser's four names are
    stubs that refuse with NotImplementedError instead of computing."""
    assert set(REFERENCE_NAMES) <= set(ng.__all__)
    assert all(hasattr(ng, n) for n in ng.__all__)
    for name in ("gptq_quantize", "quantize_model_gptq", "find_decoder_blocks",
                 "HessianAccumulator"):
        with pytest.raises(NotImplementedError, match="GPTQ"):
            getattr(ng, name)(None)


def test_extension_exposes_the_reference_module_functions():
    """``extension()`` offers the reference module's tensor-level functions
    (csrc/bindings.cpp:11-22) with the same argument names and defaults."""
    import inspect  # noqa: PLC0415

    ext = ng.extension()
    sig = inspect.signature(ext.gemv_w4a16)
    assert list(sig.parameters) == ["X", "Wq", "S", "group_size", "version", "splits_override",
                                    "threads_override"]
    assert sig.parameters["version"].default == 4
    assert inspect.signature(ext.gemm_w4a16).parameters["version"].default == 6
    assert inspect.signature(ext.dequant_w4).parameters["fast"].default is True
    X, qw = _cpu_case()
    with pytest.raises(RuntimeError, match="GPU"):
        ext.gemv_w4a16(X, qw.qweight, qw.scales, 128)
    with pytest.raises(RuntimeError, match="GPU"):
        ext.dequant_w4(qw.qweight, qw.scales, 128)


def fused(ext, M, K, N, g=128, epilogue=1, bias=P, wq_rows=None, s_rows=None, s_cols=None, ptr=P,
          norm=None, eps=1e-5):
    wq_rows = K // 8 if wq_rows is None else wq_rows
    s_rows = K // g if s_rows is None else s_rows
    s_cols = N if s_cols is None else s_cols
    return ext.matmul_fused(ptr, M, K, ptr, wq_rows, N, ptr, s_rows, s_cols, g, epilogue, bias, norm,
                            eps, ptr, None, 0, None)


@pytest.mark.parametrize("kwargs,needle", [
    (dict(M=129, K=256, N=128), "M <= 128"),
    (dict(M=4, K=256, N=128, epilogue=3), "epilogue"),
    (dict(M=4, K=256, N=80, epilogue=2), "multiple of 32"),
    (dict(M=4, K=256, N=130, epilogue=0), "multiple of 4"),
    (dict(M=4, K=256, N=128, bias=None), "null bias"),
    (dict(M=4, K=256, N=128, wq_rows=31), "packed weight rows"),
    (dict(M=4, K=256, N=128, s_cols=132), "scale columns"),
    (dict(M=4, K=0, N=128), "K and N must be positive"),
    (dict(M=4, K=256, N=128, ptr=P + 8), "aligned"),
    (dict(M=9, K=256, N=128, norm=P), "fused RMSNorm supports M <= 8"),
    (dict(M=1, K=16384 + 128, N=128, norm=P), "K <= 16384"),
    (dict(M=8, K=8192, N=128, norm=P), "above 64 KiB"),
    (dict(M=1, K=256, N=128, norm=P + 8), "norm weight must be 16-byte aligned"),
    (dict(M=1, K=256, N=128, norm=P, eps=-1.0), "norm eps"),
])
def test_fused_rejections(kwargs, needle):
    ext = ng.extension()
    assert fused(ext, **kwargs) == INVALID
    assert needle in ext.last_error()


def test_fused_workspace_matches_streaming_plan():
    """The fused entry runs the streaming kernel's plan: the same workspace as
    nibble_gemm_w4a16 wherever that streams too (M <= 32, and 33..128 rows
    whose weight passes stay under 48 MiB), and as nibble_gemv_w4a16 v4 for
    M <= 8.  Batches of 33..128 rows over large weights take tiles in
    nibble_gemm_w4a16 but still stream in the fused entry."""
    ext = ng.extension()
    for M, K, N in [(1, 4096, 14336), (1, 14336, 4096), (8, 14336, 512), (32, 14336, 4096),
                    (33, 4096, 4096), (128, 8192, 1024)]:
        assert ext.matmul_fused_workspace_bytes(M, K, N, 128, None) == \
            ext.gemm_workspace_bytes(M, K, N, 128, 6, None), (M, K, N)
    assert ext.matmul_fused_workspace_bytes(1, 14336, 4096, 128, None) == \
        ext.gemv_workspace_bytes(1, 14336, 4096, 128, 4, 0, 0, None)
    assert ext.matmul_fused_workspace_bytes(129, 4096, 4096, 128, None) == (0, 0)
    assert ext.matmul_fused_workspace_bytes(33, 14336, 4096, 128, None) != \
        ext.gemm_workspace_bytes(33, 14336, 4096, 128, 6, None)


def test_gemm_streams_query():
    """nibble_gemm_streams names the plan nibble_gemm_w4a16 takes: streaming
    for M <= 32, for 33..64 rows whose one 64-row block makes one round of
    the CUs, and for 33..128 rows whose 32-row weight passes move under
    48 MiB; tiles otherwise (where the fused entry's plan differs from
    gemm's)."""
    ext = ng.extension()
    for M, K, N, g, streams in [(1, 4096, 14336, 128, True), (32, 14336, 4096, 128, True),
                                (33, 14336, 4096, 128, True), (33, 4096, 4096, 128, True),
                                (64, 4096, 14336, 128, True), (65, 4096, 14336, 128, False),
                                (40, 4096, 28672, 128, False), (128, 4096, 6144, 64, False),
                                (64, 4096, 6144, 128, True), (128, 8192, 1024, 128, True),
                                (129, 4096, 4096, 128, False), (8, 4096, 4096, 32, False),
                                (8, 4096, 4098, 128, False), (0, 4096, 4096, 128, False)]:
        assert ext.gemm_streams(M, K, N, g) is streams, (M, K, N, g)
        if streams:
            fused = ext.matmul_fused_workspace_bytes(M, K, N, g, None)
            gemm = ext.gemm_workspace_bytes(M, K, N, g, 6, None)
            assert fused[0] >= gemm[0] and fused[1] >= gemm[1], (M, K, N, g)
            if 16 < M <= 32:
                assert fused == gemm, (M, K, N, g)


def test_gemm_streams_agrees_with_the_plans():
    """Over random batch shapes: where nibble_gemm_streams says the GEMM
    streams, the fused entry's workspace covers the GEMM's (it answers for
    the split kernel's plan and the GEMM's, so one buffer serves every
    epilogue; equal for 17..32 rows, where the batch kernel's plan is the
    larger); where it does not, the batch is 33..128 rows over passes of
    48 MiB or more (or the operands cannot stream at all)."""
    import random
    ext = ng.extension()
    rng = random.Random(7)
    for _ in range(400):
        M = rng.randint(1, 140)
        K = 128 * rng.randint(1, 128)
        N = 4 * rng.randint(1, 8000)
        g = rng.choice((64, 128))
        streams = ext.gemm_streams(M, K, N, g)
        if streams:
            fused = ext.matmul_fused_workspace_bytes(M, K, N, g, None)
            gemm = ext.gemm_workspace_bytes(M, K, N, g, 6, None)
            assert fused[0] >= gemm[0] and fused[1] >= gemm[1], (M, K, N, g)
            if 16 < M <= 32:
                assert fused == gemm, (M, K, N, g)
        else:
            assert M > 128 or (M > 32 and ((M + 31) // 32) * K * N // 2 >= 48 << 20), (M, K, N, g)


def test_last_error_is_per_thread():
    """nibble_last_error() is thread-local: a failure on one thread does not
    overwrite the message another thread is about to read."""
    import threading

    ext = ng.extension()
    first_failed, second_failed = threading.Event(), threading.Event()
    seen = {}

    def first():
        assert gemv(ext, 1, 256, 128, version=9) == INVALID
        first_failed.set()
        second_failed.wait(10)
        seen["first"] = ext.last_error()

    def second():
        first_failed.wait(10)
        assert ext.dequant(P, 32, 128, P, 2, 128, 100, 1, P, None) == INVALID
        seen["second"] = ext.last_error()
        second_failed.set()

    threads = [threading.Thread(target=first), threading.Thread(target=second)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(20)
    assert "version" in seen["first"] and "group_size" not in seen["first"]
    assert "group_size" in seen["second"]


@pytest.mark.parametrize("seed", range(4))
def test_workspace_plans_are_self_consistent(seed):
    """Over random shapes: counters are 256-byte padded, a workspace exists
    exactly when there are counters, and what follows the counters is whole
    fp32 [splits, M, N] partials with 2 to 16 (streaming plans: gemv, and
    gemm up to 128 rows) or 2 to 4 (tiled gemm) splits."""
    import random

    rng = random.Random(seed)
    ext = ng.extension()
    for _ in range(200):
        g = rng.choice([64, 128])
        K = g * rng.randint(1, 256)
        N = 4 * rng.randint(1, 8192)
        for M, kind in ((rng.randint(1, 8), "gemv"), (rng.randint(9, 4096), "gemm")):
            if kind == "gemv":
                ws, cb = ext.gemv_workspace_bytes(M, K, N, g, 4, 0, 0, None)
                max_splits = 16
            else:
                ws, cb = ext.gemm_workspace_bytes(M, K, N, g, rng.choice([6, 7]), None)
                max_splits = 16 if M <= 128 else 4  # M <= 128 streams, as gemv
            assert cb % 256 == 0 and (ws == 0) == (cb == 0), (kind, M, K, N, g, ws, cb)
            if ws:
                body = ws - cb
                assert body % (4 * M * N) == 0, (kind, M, K, N, g, ws, cb)
                assert 2 <= body // (4 * M * N) <= max_splits, (kind, M, K, N, g, ws, cb)
