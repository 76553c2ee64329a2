"""Kernel entry points and the drop-in ``QuantLinear``.

Mirrors ``python/nibblegemm/ops.py`` of arvindcr4/nibblegemm (names, defaults,
dispatch rule and error types), over the C ABI in ``include/nibblegemm_amd.h``
instead of a pybind11 torch extension:

* tensors are validated here exactly as the reference's ``TORCH_CHECK``s did
  (dtype, device, contiguity, rank: ``RuntimeError``); shape checks run inside
  the library and come back as a status that is raised as ``RuntimeError``;
* outputs are allocated here with torch on X's device (Wq's for ``dequant``),
  as the reference allocated them in C++;
* kernels launch on torch's current stream of that device, so calls compose
  with torch ops and can be recorded into CUDA/HIP graphs;
* the split-K workspace of the split kernel comes from a cache of zeroed
  buffers keyed by (device, stream, graph capture, counter-region size): the
  kernel returns its counter region to zero at the end of every call, so a
  buffer is zeroed once and then reused.  Inside a graph capture the first call
  allocates and zeroes a buffer for that capture from the graph's private
  memory pool, so the zeroing is part of the graph and every replay starts
  from zero.  The cache holds a capture's buffers only while that capture is
  in progress: the first call from another capture, or outside any, drops
  them, and the graph's pool keeps their memory until the graph is destroyed.
  (Graphs that share one memory pool must not be replayed concurrently with
  each other -- PyTorch's own condition for sharing a pool.)
"""
from __future__ import annotations

import ctypes
import threading
from typing import Dict, Optional, Tuple

import torch

from . import _native
from .quant import (SWIGLU_BLOCK, QuantizedWeight, StripMajorWeight,  # noqa: F401
                    from_strip_major, quantize, split_swiglu)

#: Batch sizes at or below this go to the bandwidth-bound decode kernel
#: (reference ops.py:30).
DECODE_MAX_M = 8

_lock = threading.Lock()
_workspaces: Dict[Tuple[int, int, int, int], torch.Tensor] = {}
_capture_entries = 0  # cached buffers that belong to a graph capture
_ws_plan: Dict[tuple, Tuple[int, int]] = {}

_get_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


class _Extension:
    """What ``extension()`` returns: the reference extension module's three
    tensor-level functions, with its argument names and defaults
    (csrc/bindings.cpp:11-22), over the C ABI.  Attributes it does not define
    (the pointer-level calls ``gemv``, ``gemm``, ``dequant``,
    ``gemv_workspace_bytes``, ``last_error``, ``abi_version``) resolve to the
    CPython binding."""

    def __init__(self, binding):
        self._binding = binding

    def __getattr__(self, name):
        return getattr(self._binding, name)

    @staticmethod
    def _qw(Wq: torch.Tensor, S: torch.Tensor, group_size: int) -> QuantizedWeight:
        rows = Wq.shape[0] if Wq.dim() == 2 else 0
        cols = Wq.shape[1] if Wq.dim() == 2 else 0
        return QuantizedWeight(Wq, S, int(group_size), rows * 8, cols)

    def gemv_w4a16(self, X, Wq, S, group_size, version=4, splits_override=0, threads_override=0):
        return gemv(X, self._qw(Wq, S, group_size), version, splits_override, threads_override)

    def gemm_w4a16(self, X, Wq, S, group_size, version=6):
        return gemm(X, self._qw(Wq, S, group_size), version)

    def dequant_w4(self, Wq, S, group_size, fast=True):
        return dequant(self._qw(Wq, S, group_size), fast)


_extension: Optional[_Extension] = None


def extension() -> _Extension:
    """The loaded native extension (reference ops.py:33-56 JIT-built it on first
    use; this package is built in-tree ahead of time and only loads it).
    Raises RuntimeError, naming the build command, when it is not built."""
    global _extension
    if _extension is None:
        _extension = _Extension(_native.binding())
    return _extension


def _bind():
    return _native.binding()


def _raise(rc: int, ext) -> None:
    raise RuntimeError(f"nibblegemm_amd: {ext.last_error()} (status {rc})")


def _stream(device: torch.device) -> int:
    if _get_raw_stream is not None:
        return _get_raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _check_matmul_inputs(X: torch.Tensor, Wq: torch.Tensor, S: torch.Tensor) -> None:
    """The dtype/device/layout half of check_inputs (reference
    csrc/gemv_w4a16.cu:251-258, csrc/gemm_w4a16.cu:381-386)."""
    if not (X.is_cuda and Wq.is_cuda and S.is_cuda):
        raise RuntimeError("all tensors must live on the GPU")
    if X.dtype != torch.float16:
        raise RuntimeError("activations must be fp16")
    if S.dtype != torch.float16:
        raise RuntimeError("scales must be fp16")
    if Wq.dtype != torch.int32:
        raise RuntimeError("packed weights must be int32")
    if not (X.is_contiguous() and Wq.is_contiguous() and S.is_contiguous()):
        raise RuntimeError("inputs must be contiguous")
    if X.dim() != 2 or Wq.dim() != 2 or S.dim() != 2:
        raise RuntimeError("expected 2-D inputs")
    if not (X.device == Wq.device == S.device):
        raise RuntimeError("all tensors must live on the same device")


_hip = None


def _capture_id(stream: int) -> int:
    """0 outside graph capture, else the HIP capture id of ``stream``."""
    if not torch.cuda.is_current_stream_capturing():
        return 0
    global _hip
    if _hip is None:
        lib = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch already loaded
        lib.hipStreamGetCaptureInfo.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int),
                                                ctypes.POINTER(ctypes.c_ulonglong)]
        lib.hipStreamGetCaptureInfo.restype = ctypes.c_int
        _hip = lib
    status, cid = ctypes.c_int(0), ctypes.c_ulonglong(0)
    rc = _hip.hipStreamGetCaptureInfo(ctypes.c_void_p(stream), ctypes.byref(status), ctypes.byref(cid))
    if rc != 0:
        raise RuntimeError(f"hipStreamGetCaptureInfo failed ({rc})")
    return int(cid.value) or -1


def _workspace(plan: Tuple[int, int], device: torch.device,
               stream: int) -> Tuple[Optional[torch.Tensor], int]:
    """A zeroed buffer of at least ``plan[0]`` bytes whose leading
    ``plan[1]`` bytes (split-K counters) are zero; None if no bytes needed."""
    global _capture_entries
    nbytes, counter_bytes = plan
    if nbytes == 0:
        return None, 0
    # One buffer per counter-region size: a plan's fp32 partials start right
    # after its counters, so a plan with fewer counters would overwrite the
    # (zero) counters of a plan with more if they shared a buffer.
    capture = _capture_id(stream)
    wkey = (device.index, stream, capture, counter_bytes)
    buf = _workspaces.get(wkey)
    if buf is None or buf.numel() < nbytes:
        with _lock:
            _drop_ended_captures(capture)
            buf = _workspaces.get(wkey)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 20)
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                _workspaces[wkey] = buf
                if capture != 0:
                    _capture_entries += 1
    elif capture == 0 and _capture_entries:
        with _lock:
            _drop_ended_captures(0)
    return buf, buf.numel()


def _drop_ended_captures(current: int) -> None:
    """Forget the buffers of every capture other than ``current`` (called
    under ``_lock``).  Calls are made from one capture at a time, so a call
    from elsewhere means those captures have ended; their memory belongs to
    their graphs' pools, which free it with the graphs."""
    global _capture_entries
    if not _capture_entries:
        return
    for key in [k for k in _workspaces if k[2] not in (0, current)]:
        del _workspaces[key]
    _capture_entries = sum(1 for k in _workspaces if k[2] != 0)


def release_workspaces() -> None:
    """Drop every cached split-K workspace (eager and capture buffers alike);
    later calls allocate and zero fresh ones."""
    global _capture_entries
    with _lock:
        _workspaces.clear()
        _capture_entries = 0


def _gemv_workspace(ext, device: torch.device, stream: int, M: int, K: int, N: int, g: int,
                    version: int, splits: int, threads: int) -> Tuple[Optional[torch.Tensor], int]:
    key = ("gemv", M, K, N, g, version, splits, threads)
    plan = _ws_plan.get(key)
    if plan is None:
        plan = ext.gemv_workspace_bytes(M, K, N, g, version, splits, threads, stream)
        _ws_plan[key] = plan
    return _workspace(plan, device, stream)


def _gemm_workspace(ext, device: torch.device, stream: int, M: int, K: int, N: int, g: int,
                    version: int) -> Tuple[Optional[torch.Tensor], int]:
    key = ("gemm", M, K, N, g, version)
    plan = _ws_plan.get(key)
    if plan is None:
        plan = ext.gemm_workspace_bytes(M, K, N, g, version, stream)
        _ws_plan[key] = plan
    return _workspace(plan, device, stream)


def dequant(qw: QuantizedWeight, fast: bool = True) -> torch.Tensor:
    """Expand packed INT4 to a dense ``[K, N]`` fp16 matrix on the device
    (reference ops.py:59-61 -> csrc/dequant_kernel.cu:48-74).  A
    :class:`StripMajorWeight` gives the same matrix as the packed weight it
    was made from."""
    ext = _bind()
    Wq, S = qw.qweight, qw.scales
    if isinstance(qw, StripMajorWeight):
        _check_strip_weight(qw)
        out = torch.empty((qw.K, qw.N), dtype=torch.float16, device=Wq.device)
        rc = ext.dequant_strip_major(Wq.data_ptr(), S.data_ptr(), qw.K, qw.N, qw.group_size,
                                     qw.strip_cols, 1 if fast else 0, out.data_ptr(),
                                     _stream(Wq.device))
        if rc:
            _raise(rc, ext)
        return out
    if not (Wq.is_cuda and S.is_cuda):
        raise RuntimeError("tensors must live on the GPU")
    if Wq.dtype != torch.int32:
        raise RuntimeError("packed weights must be int32")
    if S.dtype != torch.float16:
        raise RuntimeError("scales must be fp16")
    if not (Wq.is_contiguous() and S.is_contiguous()):
        raise RuntimeError("inputs must be contiguous")
    if Wq.dim() != 2 or S.dim() != 2:
        raise RuntimeError("expected 2-D inputs")
    rows, N = Wq.shape
    out = torch.empty((rows * 8, N), dtype=torch.float16, device=Wq.device)
    rc = ext.dequant(Wq.data_ptr(), rows, N, S.data_ptr(), S.shape[0], S.shape[1],
                     qw.group_size, 1 if fast else 0, out.data_ptr(), _stream(Wq.device))
    if rc:
        _raise(rc, ext)
    return out


def gemv(X: torch.Tensor, qw: QuantizedWeight, version: int = 4, splits: int = 0,
         block_threads: int = 0) -> torch.Tensor:
    """Decode-regime matmul (reference ops.py:64-74).

    ``version``: 0/1 scalar fp32 kernels, 2/3 streaming kernel with one K split,
    4 (default) streaming kernel with split-K.  ``splits`` and ``block_threads``
    override the launch geometry (0 = heuristic); ``block_threads`` is 32 (run
    as one 64-lane wave, as the reference accepts it) or a multiple of the
    64-lane wave up to 1024.  Versions 3 and 4 serve M <= 8.
    """
    ext = _bind()
    Wq, S = qw.qweight, qw.scales
    _check_matmul_inputs(X, Wq, S)
    M, K = X.shape
    N = Wq.shape[1]
    dev = X.device
    stream = _stream(dev)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    ws, ws_bytes = None, 0
    if version == 4 and 0 < M <= DECODE_MAX_M:
        ws, ws_bytes = _gemv_workspace(ext, dev, stream, M, K, N, qw.group_size, version, splits,
                                       block_threads)
    rc = ext.gemv(X.data_ptr(), M, K, Wq.data_ptr(), Wq.shape[0], N, S.data_ptr(), S.shape[0],
                  S.shape[1], qw.group_size, version, splits, block_threads, Y.data_ptr(),
                  ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    if rc:
        _raise(rc, ext)
    return Y


def gemm(X: torch.Tensor, qw: QuantizedWeight, version: int = 6) -> torch.Tensor:
    """Prefill-regime matmul on MFMA (reference ops.py:77-86).  ``version`` 6
    (default) or 7 select two tile shapes with identical numerics; batches of
    M <= 128 run the GEMV's weight-streaming kernel whatever the version.  A
    :class:`StripMajorWeight` runs the same plans and kernels (the same bits
    as its packed weight) from 9 rows, the strip-major GEMV below."""
    if isinstance(qw, StripMajorWeight):
        return _strip_gemm(X, qw, version)
    ext = _bind()
    Wq, S = qw.qweight, qw.scales
    _check_matmul_inputs(X, Wq, S)
    M, K = X.shape
    N = Wq.shape[1]
    dev = X.device
    stream = _stream(dev)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    ws, ws_bytes = _gemm_workspace(ext, dev, stream, M, K, N, qw.group_size, version)
    rc = ext.gemm(X.data_ptr(), M, K, Wq.data_ptr(), Wq.shape[0], N, S.data_ptr(), S.shape[0],
                  S.shape[1], qw.group_size, version, Y.data_ptr(),
                  ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    if rc:
        _raise(rc, ext)
    return Y


def strip_major_cols(K: int, N: int, group_size: int) -> int:
    """The strip width :func:`to_strip_major` picks for a ``[K, N]`` weight
    (0 when no strip-major layout fits it)."""
    return int(_bind().strip_major_cols(K, N, group_size))


def to_strip_major(qw: QuantizedWeight, strip_cols: int = 0) -> StripMajorWeight:
    """A device copy of ``qw`` in the strip-major layout of the decode GEMV
    (one permutation kernel on the current stream; same bytes again).
    ``strip_cols`` 0 picks :func:`strip_major_cols`.  The result serves
    :func:`matmul`, :func:`gemm`, :func:`dequant` and the fused ops at every
    batch size (the fused epilogues run in the kernel up to 8 rows)."""
    ext = _bind()
    Wq, S = qw.qweight, qw.scales
    if not (Wq.is_cuda and S.is_cuda):
        raise RuntimeError("tensors must live on the GPU")
    if Wq.dtype != torch.int32 or S.dtype != torch.float16:
        raise RuntimeError("packed weights must be int32 and scales fp16")
    if not (Wq.is_contiguous() and S.is_contiguous()) or Wq.dim() != 2 or S.dim() != 2:
        raise RuntimeError("expected contiguous 2-D weights and scales")
    sw = int(strip_cols) or strip_major_cols(qw.K, qw.N, qw.group_size)
    if sw == 0:
        raise ValueError(f"no strip-major layout fits K={qw.K}, N={qw.N}, "
                         f"group_size={qw.group_size}")
    if sw <= 0 or qw.N % sw:
        raise ValueError(f"N={qw.N} is not a multiple of strip_cols={sw}")
    dev = Wq.device
    Wt = torch.empty((qw.N // sw, qw.K // 8, sw), dtype=torch.int32, device=dev)
    St = torch.empty((qw.N // sw, S.shape[0], sw), dtype=torch.float16, device=dev)
    rc = ext.pack_strip_major(Wq.data_ptr(), Wq.shape[0], Wq.shape[1], S.data_ptr(), S.shape[0],
                              S.shape[1], qw.group_size, sw, Wt.data_ptr(), St.data_ptr(),
                              _stream(dev))
    if rc:
        _raise(rc, ext)
    return StripMajorWeight(Wt, St, qw.group_size, qw.K, qw.N, sw)


def _check_strip_weight(w: StripMajorWeight) -> None:
    Wt, St = w.qweight, w.scales
    if not (Wt.is_cuda and St.is_cuda):
        raise RuntimeError("tensors must live on the GPU")
    if Wt.dtype != torch.int32 or St.dtype != torch.float16:
        raise RuntimeError("strip-major weights must be int32 and scales fp16")
    if not (Wt.is_contiguous() and St.is_contiguous()):
        raise RuntimeError("inputs must be contiguous")


def _strip_gemm(X: torch.Tensor, w: StripMajorWeight, version: int = 6) -> torch.Tensor:
    """``X @ W`` on strip-major weights: at most 8 rows through the strip-major
    GEMV, more through the packed layout's GEMM plans."""
    if X.dim() == 2 and X.size(0) <= DECODE_MAX_M:
        return _strip_gemv(X, w, 0, None, w.N)
    ext = _bind()
    _check_strip_weight(w)
    if not X.is_cuda:
        raise RuntimeError("all tensors must live on the GPU")
    if X.dtype != torch.float16:
        raise RuntimeError("activations must be fp16")
    if not X.is_contiguous() or X.dim() != 2:
        raise RuntimeError("activations must be a contiguous 2-D matrix")
    if X.device != w.qweight.device:
        raise RuntimeError("all tensors must live on the same device")
    M, K = X.shape
    dev = X.device
    stream = _stream(dev)
    Y = torch.empty((M, w.N), dtype=torch.float16, device=dev)
    ws, ws_bytes = _gemm_workspace(ext, dev, stream, M, w.K, w.N, w.group_size, version)
    rc = ext.gemm_strip_major(X.data_ptr(), M, K, w.qweight.data_ptr(), w.scales.data_ptr(), w.K,
                              w.N, w.group_size, w.strip_cols, version, Y.data_ptr(),
                              ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    if rc:
        _raise(rc, ext)
    return Y


def _strip_gemv(X: torch.Tensor, w: StripMajorWeight, epilogue: int,
                bias: Optional[torch.Tensor], n_out: int,
                norm: Optional[Tuple[torch.Tensor, float]] = None) -> torch.Tensor:
    ext = _bind()
    Wt, St = w.qweight, w.scales
    if not (X.is_cuda and Wt.is_cuda and St.is_cuda):
        raise RuntimeError("all tensors must live on the GPU")
    if X.dtype != torch.float16:
        raise RuntimeError("activations must be fp16")
    if Wt.dtype != torch.int32 or St.dtype != torch.float16:
        raise RuntimeError("strip-major weights must be int32 and scales fp16")
    if not (X.is_contiguous() and Wt.is_contiguous() and St.is_contiguous()):
        raise RuntimeError("inputs must be contiguous")
    if not (X.device == Wt.device == St.device):
        raise RuntimeError("all tensors must live on the same device")
    M, K = X.shape
    if M > DECODE_MAX_M:
        raise ValueError(f"strip-major weights serve batches of at most {DECODE_MAX_M} rows, "
                         f"got {M}; multiply larger batches with the packed weight")
    dev = X.device
    Y = torch.empty((M, n_out), dtype=torch.float16, device=dev)
    rc = ext.gemv_strip_major(X.data_ptr(), M, K, Wt.data_ptr(), St.data_ptr(), w.K, w.N,
                              w.group_size, w.strip_cols, epilogue,
                              bias.data_ptr() if bias is not None else None,
                              norm[0].data_ptr() if norm is not None else None,
                              float(norm[1]) if norm is not None else 0.0, Y.data_ptr(),
                              _stream(dev))
    if rc:
        _raise(rc, ext)
    return Y


def matmul(X: torch.Tensor, qw, splits: int = 0, block_threads: int = 0) -> torch.Tensor:
    """``X @ dequant(qw)``, dispatching on batch size (reference ops.py:89-104):
    M <= DECODE_MAX_M goes to ``gemv(version=4)``, larger M to ``gemm``.  A
    :class:`StripMajorWeight` (M <= 8 only) runs the strip-major GEMV."""
    if X.dim() != 2:
        raise ValueError(f"expected a 2-D activation matrix, got {tuple(X.shape)}")
    if X.size(1) != qw.K:
        raise ValueError(f"K mismatch: activations have {X.size(1)}, weights have {qw.K}")
    if isinstance(qw, StripMajorWeight):
        if splits or block_threads:
            raise ValueError("strip-major weights take no splits / block_threads override")
        return _strip_gemm(X, qw)
    if X.size(0) <= DECODE_MAX_M:
        return gemv(X, qw, version=4, splits=splits, block_threads=block_threads)
    return gemm(X, qw)


#: Largest batch the fused-epilogue entry point takes (the streaming kernel's).
FUSED_MAX_M = 128


def _fused_workspace(ext, device: torch.device, stream: int, M: int, K: int, N: int,
                     g: int) -> Tuple[Optional[torch.Tensor], int]:
    key = ("fused", M, K, N, g)
    plan = _ws_plan.get(key)
    if plan is None:
        plan = ext.matmul_fused_workspace_bytes(M, K, N, g, stream)
        _ws_plan[key] = plan
    return _workspace(plan, device, stream)


def _fusable(X: torch.Tensor, qw: QuantizedWeight) -> bool:
    """Whether the fused-epilogue launch takes these operands and computes
    the product with ``matmul``'s bits (else the caller composes the same
    arithmetic from separate ops).  The fused launch streams; ``matmul``
    takes tiles for batches of 33..128 rows over large weights, so those
    compose."""
    return (X.dim() == 2 and X.is_cuda and 1 <= X.size(0) <= FUSED_MAX_M and qw.N % 4 == 0
            and X.is_contiguous() and X.data_ptr() % 16 == 0
            and qw.qweight.data_ptr() % 16 == 0 and qw.scales.data_ptr() % 8 == 0
            and _bind().gemm_streams(X.size(0), qw.K, qw.N, qw.group_size))


def _fused(X: torch.Tensor, qw: QuantizedWeight, epilogue: int, bias: Optional[torch.Tensor],
           n_out: int, norm: Optional[Tuple[torch.Tensor, float]] = None) -> torch.Tensor:
    ext = _bind()
    Wq, S = qw.qweight, qw.scales
    _check_matmul_inputs(X, Wq, S)
    M, K = X.shape
    N = Wq.shape[1]
    dev = X.device
    stream = _stream(dev)
    Y = torch.empty((M, n_out), dtype=torch.float16, device=dev)
    ws, ws_bytes = _fused_workspace(ext, dev, stream, M, K, N, qw.group_size)
    rc = ext.matmul_fused(X.data_ptr(), M, K, Wq.data_ptr(), Wq.shape[0], N, S.data_ptr(),
                          S.shape[0], S.shape[1], qw.group_size, epilogue,
                          bias.data_ptr() if bias is not None else None,
                          norm[0].data_ptr() if norm is not None else None,
                          float(norm[1]) if norm is not None else 0.0, Y.data_ptr(),
                          ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    if rc:
        _raise(rc, ext)
    return Y


def _check_2d(X: torch.Tensor, qw: QuantizedWeight) -> None:
    if X.dim() != 2:
        raise ValueError(f"expected a 2-D activation matrix, got {tuple(X.shape)}")
    if X.size(1) != qw.K:
        raise ValueError(f"K mismatch: activations have {X.size(1)}, weights have {qw.K}")


def matmul_bias(X: torch.Tensor, qw: QuantizedWeight, bias: torch.Tensor) -> torch.Tensor:
    """``matmul(X, qw) + bias`` -- the arithmetic of the reference's
    ``QuantLinear`` with a bias (ops.py:131-135): the fp16 product, then the
    bias added in fp16.  An fp16 bias with M <= 128 runs as one launch (the
    bias added in the kernel's epilogue, same bits); other cases run the two
    ops."""
    _check_2d(X, qw)
    fp16_bias = (bias.dtype == torch.float16 and bias.dim() == 1 and bias.numel() == qw.N
                 and bias.device == X.device and bias.is_contiguous())
    if isinstance(qw, StripMajorWeight):
        if fp16_bias and X.size(0) <= DECODE_MAX_M:
            return _strip_gemv(X, qw, 1, bias, qw.N)
    elif fp16_bias and _fusable(X, qw):
        return _fused(X, qw, 1, bias, qw.N)
    return matmul(X, qw) + bias


def matmul_swiglu(X: torch.Tensor, qw: QuantizedWeight) -> torch.Tensor:
    """``silu(X @ W_gate) * (X @ W_up)`` for ``qw = interleave_swiglu(gate,
    up)``, with the fp16 roundings of the unfused ops (the two products,
    silu, then the product).  M <= 128 runs as one launch; so does a
    strip-major weight whose strips hold whole gate|up block pairs (at least
    32 columns), while narrower strips compose the same arithmetic from the
    plain product."""
    _check_2d(X, qw)
    if qw.N % (2 * SWIGLU_BLOCK):
        raise ValueError(f"N={qw.N} is not an interleaved gate|up weight (multiple of 32)")
    if isinstance(qw, StripMajorWeight):
        if qw.strip_cols >= 2 * SWIGLU_BLOCK and X.size(0) <= DECODE_MAX_M:
            return _strip_gemv(X, qw, 2, None, qw.N // 2)
        gate, up = split_swiglu(_strip_gemm(X, qw))
        return torch.nn.functional.silu(gate) * up
    if _fusable(X, qw):
        return _fused(X, qw, 2, None, qw.N // 2)
    gate, up = split_swiglu(matmul(X, qw))
    return torch.nn.functional.silu(gate) * up


#: Largest batch ``rmsnorm_matmul`` runs as one launch.  The kernels take the
#: RMSNorm prologue up to 8 rows, but from 4 rows the two launches are faster
#: (MI355X, strip-major weights, graph replay, fused vs composed): 4096 x 6144
#: M = 1 / 3 / 4 / 8 5.9 / 7.1 / 7.6 / 9.9 us vs 6.8 / 7.2 / 7.4 / 7.7;
#: 4096 x 28672 SwiGLU M = 1 / 4 / 8 12.0 / 15.4 / 30.0 vs 14.4 / 15.0 /
#: 15.5 (at 8 rows the staged norm weight leaves room for one workgroup per
#: CU instead of two).
NORM_FUSED_MAX_M = 3
NORM_FUSED_MAX_K = 16384


def rmsnorm_matmul(X: torch.Tensor, norm_weight: torch.Tensor, qw: QuantizedWeight,
                   eps: float = 1e-5, *, bias: Optional[torch.Tensor] = None,
                   swiglu: bool = False) -> torch.Tensor:
    """``matmul(rmsnorm(X, norm_weight, eps), qw)``, optionally through the
    bias or SwiGLU epilogue (:func:`matmul_bias`, :func:`matmul_swiglu`).

    For M <= 3 and K <= 16384 (the normalised rows fitting 64 KiB) this is one
    launch: the streaming kernel normalises the rows itself, with the
    RMSNorm kernel's arithmetic, so the result has the bits of the two-step
    composition, which runs otherwise (:data:`NORM_FUSED_MAX_M`)."""
    _check_2d(X, qw)
    if bias is not None and swiglu:
        raise ValueError("bias and swiglu epilogues are exclusive")
    if swiglu and qw.N % (2 * SWIGLU_BLOCK):
        raise ValueError(f"N={qw.N} is not an interleaved gate|up weight (multiple of 32)")
    M, K = X.shape
    mt = 1 if M <= 1 else 2 if M <= 2 else 4 if M <= 4 else 8
    strip = isinstance(qw, StripMajorWeight)
    fusable = (X.dim() == 2 and X.is_cuda and X.is_contiguous()) if strip else _fusable(X, qw)
    if swiglu and strip and qw.strip_cols < 2 * SWIGLU_BLOCK:
        fusable = False  # the SwiGLU epilogue needs whole gate|up block pairs per strip
    if (fusable and M <= NORM_FUSED_MAX_M and K <= NORM_FUSED_MAX_K and mt * K * 2 <= 65536
            and norm_weight.dtype == torch.float16 and norm_weight.is_contiguous()
            and norm_weight.device == X.device and norm_weight.numel() == K
            and norm_weight.data_ptr() % 16 == 0 and X.dtype == torch.float16
            and (bias is None or (bias.dtype == torch.float16 and bias.dim() == 1
                                  and bias.numel() == qw.N and bias.is_contiguous()
                                  and bias.device == X.device))):
        run = _strip_gemv if strip else _fused
        if swiglu:
            return run(X, qw, 2, None, qw.N // 2, (norm_weight, eps))
        return run(X, qw, 1 if bias is not None else 0, bias, qw.N, (norm_weight, eps))
    from .glue import rmsnorm  # noqa: PLC0415  (glue imports this module)
    a = rmsnorm(X, norm_weight, eps)
    if swiglu:
        return matmul_swiglu(a, qw)
    return matmul_bias(a, qw, bias) if bias is not None else matmul(a, qw)


class QuantLinear(torch.nn.Module):
    """An ``nn.Linear`` whose weight is packed INT4 (reference ops.py:107-135).

    The module holds three buffers under the reference's names -- ``qweight``
    (int32 ``[in/8, out]``), ``scales`` (fp16 ``[in/G, out]``) and ``bias``
    (or None) -- so state dicts move between the two packages unchanged.
    ``forward`` flattens leading dimensions, multiplies through
    :func:`matmul` and adds the bias; an fp16 bias is added inside the
    matmul's output stage where the kernel supports it (same bits as a
    separate fp16 add).

    :meth:`prepare_decode` converts the weight, in place, to the strip-major
    layout (:func:`to_strip_major`), which every batch size reads: at most 8
    rows through the strip-major GEMV (the fast decode path), more through
    the same GEMM plans as the packed weight (the same bits).  The module
    then holds that one copy -- ``qweight`` ``[out/SW, in/8, SW]``,
    ``scales`` ``[out/SW, in/G, SW]``, ``strip_cols`` = SW -- and converts at
    the state-dict boundary: ``state_dict()`` returns the packed tensors and
    ``load_state_dict()`` takes packed tensors.  :meth:`release_decode`
    converts back."""

    def __init__(self, qw: QuantizedWeight, bias: Optional[torch.Tensor] = None):
        super().__init__()
        self.group_size = qw.group_size
        self.K = qw.K
        self.N = qw.N
        for name, tensor in (("qweight", qw.qweight), ("scales", qw.scales), ("bias", bias)):
            self.register_buffer(name, tensor)
        self.strip_cols = 0

    def prepare_decode(self, strip_cols: int = 0) -> "QuantLinear":
        """Convert the weight to the strip-major layout on its GPU, in place
        (``strip_cols`` 0 picks :func:`strip_major_cols`, the launches'
        width; :func:`nibblegemm_amd.chain.chain_strip_cols` gives the width
        a decode chain streams fastest); returns the module.  The packed copy
        is released once converted."""
        if self.strip_cols:
            if strip_cols in (0, self.strip_cols):
                return self
            self.release_decode()
        sm = to_strip_major(self._qw(), strip_cols)
        self.qweight, self.scales, self.strip_cols = sm.qweight, sm.scales, sm.strip_cols
        return self

    def release_decode(self) -> "QuantLinear":
        """Convert a strip-major weight back to the packed layout, in place."""
        if self.strip_cols:
            qw = self._packed()
            self.qweight, self.scales, self.strip_cols = qw.qweight, qw.scales, 0
        return self

    def _packed(self) -> QuantizedWeight:
        """The packed form of the weight (a converted copy when strip-major)."""
        if not self.strip_cols:
            return self._qw()
        return from_strip_major(self._qw())

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        if self.strip_cols:
            qw = self._packed()
            destination[prefix + "qweight"] = qw.qweight
            destination[prefix + "scales"] = qw.scales

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        qk, sk = prefix + "qweight", prefix + "scales"
        if self.strip_cols and qk in state_dict and sk in state_dict:
            packed = QuantizedWeight(state_dict[qk].to(self.qweight.device).contiguous(),
                                     state_dict[sk].to(self.scales.device).contiguous(),
                                     self.group_size, self.K, self.N)
            sm = to_strip_major(packed, self.strip_cols)
            state_dict = dict(state_dict)
            state_dict[qk], state_dict[sk] = sm.qweight, sm.scales
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    @classmethod
    def from_linear(cls, linear: torch.nn.Linear, group_size: int = 128) -> "QuantLinear":
        """Quantise ``linear`` (RTN, group ``group_size``) onto its own device.
        ``nn.Linear`` keeps ``[out_features, in_features]``; the packed format
        is ``[K = in_features, N = out_features]``, hence the transpose."""
        weight_kn = linear.weight.detach().transpose(0, 1).contiguous()
        bias = None if linear.bias is None else linear.bias.detach().clone()
        return cls(quantize(weight_kn, group_size).to(linear.weight.device), bias)

    def _qw(self):
        if self.strip_cols:
            return StripMajorWeight(self.qweight, self.scales, self.group_size, self.K, self.N,
                                    self.strip_cols)
        return QuantizedWeight(self.qweight, self.scales, self.group_size, self.K, self.N)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        rows = x.reshape(-1, x.shape[-1]).contiguous()
        w = self._qw()
        y = matmul(rows, w) if self.bias is None else matmul_bias(rows, w, self.bias)
        return y.reshape(*lead, self.N)
