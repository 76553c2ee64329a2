"""nibble_gemv_w4a16_noalloc -- the decode GEMV whose split-K workspace is the
library's static device scratch -- called through the C ABI and compared with
nibble_gemv_w4a16 given a caller workspace (through the package's ``gemv``).
Both run the same plan and kernels, so the results must be equal to the bit.

The calls come in pairs, the second smaller than the first, because every call
on a GPU reuses the same scratch: its counters must have been left at zero and
stale partials of the larger call must not leak into the smaller one.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

import nibblegemm_amd as ng
from nibblegemm_amd import _native
from cases import synthetic

pytestmark = pytest.mark.gpu

_lib = ctypes.CDLL(_native.LIBRARY_PATH)
_fn = _lib.nibble_gemv_w4a16_noalloc
_fn.restype = ctypes.c_int
_fn.argtypes = ([ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64] * 3
                + [ctypes.c_int64] * 4 + [ctypes.c_void_p, ctypes.c_void_p])
_lib.nibble_last_error.restype = ctypes.c_char_p
_SHAPES_ARGS = None


def noalloc(X: torch.Tensor, qw: ng.QuantizedWeight, version: int = 4, splits: int = 0,
            threads: int = 0) -> torch.Tensor:
    M, K = X.shape
    Y = torch.empty((M, qw.N), dtype=torch.float16, device=X.device)
    stream = torch.cuda.current_stream().cuda_stream
    rc = _fn(X.data_ptr(), M, K, qw.qweight.data_ptr(), qw.qweight.shape[0], qw.N,
             qw.scales.data_ptr(), qw.scales.shape[0], qw.N, qw.group_size, version, splits,
             threads, Y.data_ptr(), stream)
    if rc:
        raise RuntimeError(f"status {rc}: {_lib.nibble_last_error().decode()}")
    return Y


def case(M: int, K: int, N: int, seed: int):
    _, _, _, Xd, qw = synthetic(M, K, N, 128, seed=seed)
    return Xd, qw


@pytest.mark.parametrize("first,second,splits", [
    ((4, 14336, 4096), (1, 14336, 1024), 0),  # the default plan splits K = 14336 four ways
    ((8, 4096, 2048), (2, 2048, 512), 8),      # explicit split counts: 8 then 8 of 16 groups
    ((3, 8192, 3072), (1, 1024, 256), 2),
])
def test_matches_the_workspace_entry_point_on_two_calls(first, second, splits):
    for i, (M, K, N) in enumerate((first, second)):
        X, qw = case(M, K, N, seed=10 * i + M)
        ws_bytes, _ = ng.extension().gemv_workspace_bytes(M, K, N, 128, 4, splits, 0, None)
        assert ws_bytes > 0, "the case must exercise the split-K scratch"
        want = ng.gemv(X, qw, version=4, splits=splits)
        got = noalloc(X, qw, splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, K, N, splits)


def test_plans_without_a_split_need_no_scratch():
    for M, K, N in [(1, 4096, 4096), (5, 8192, 1024)]:
        X, qw = case(M, K, N, seed=3)
        assert ng.extension().gemv_workspace_bytes(M, K, N, 128, 4, 0, 0, None) == (0, 0)
        assert torch.equal(noalloc(X, qw), ng.gemv(X, qw))
    X, qw = case(2, 1024, 512, seed=4)
    for version in (0, 1, 2, 3):
        assert torch.equal(noalloc(X, qw, version=version), ng.gemv(X, qw, version=version))


def test_graph_replays_match_eager():
    X, qw = case(2, 14336, 4096, seed=5)
    eager = ng.gemv(X, qw)
    noalloc(X, qw)  # scratch set up outside the capture
    torch.cuda.synchronize()
    out = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        out.copy_(noalloc(X, qw))
    for _ in range(3):
        out.zero_()
        ng.gemv(*case(1, 14336, 1024, seed=6))  # other eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_first_split_call_under_capture_is_refused_in_a_fresh_process():
    """The scratch of a GPU is set up by its first split-K call (counters
    cleared, then the address published); that call cannot be recorded into a
    graph, so in a process that has made none, a capture of one is refused
    with a clear error, and an eager call afterwards sets up and computes
    the workspace entry point's bits.  Runs in a child process: this one has
    set its scratch up already."""
    import os  # noqa: PLC0415
    import subprocess  # noqa: PLC0415
    import sys  # noqa: PLC0415

    code = r"""
import sys, torch
sys.path[:0] = sys.argv[1:4]  # tests/, oracle/ (before the root: its module, not the folder), root
import test_zz_no_alloc as T
import nibblegemm_amd as ng
X, qw = T.case(2, 14336, 4096, seed=5)
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
g = torch.cuda.CUDAGraph()
refused = False
try:
    with torch.cuda.graph(g, stream=side):
        T.noalloc(X, qw)
except RuntimeError as e:
    refused = "graph capture" in str(e)
torch.cuda.synchronize()
got = T.noalloc(X, qw)
ok = torch.equal(got, ng.gemv(X, qw))
print("RESULT", refused, ok, flush=True)
"""
    tests_dir = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(tests_dir)
    r = subprocess.run([sys.executable, "-c", code, tests_dir, os.path.join(root, "oracle"), root],
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "RESULT True True" in r.stdout, (r.stdout[-500:], r.stderr[-2000:])


def test_rejects_plans_beyond_the_scratch():
    X, qw = case(8, 4096, 8192, seed=7)
    with pytest.raises(RuntimeError, match="static scratch"):
        noalloc(X, qw, splits=16)  # 16 x 8 x 8192 fp32 partials = 4 MiB
    # the workspace entry point still serves it
    assert torch.isfinite(ng.gemv(X, qw, splits=16).float()).all()
