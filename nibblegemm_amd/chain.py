"""Persistent decode chains: many decode GEMVs in ONE launch.

No counterpart in the reference, whose batch-1 decode step is one launch per
projection (bench/bench_model.py:70-86) and whose optimisation log names
fewer launches as the fix for launch-bound small projections
(docs/OPTIMIZATION_LOG.md:159-163).  A :class:`DecodeChain` is a fixed list of
stages -- ``Y = X @ W`` on a :class:`~nibblegemm_amd.quant.StripMajorWeight`
or on the reference's packed :class:`~nibblegemm_amd.quant.QuantizedWeight`
unconverted, optionally with the bias or SwiGLU epilogue -- where a stage may
name an earlier one (``after``) that must finish before it reads its inputs.  One
:meth:`DecodeChain.run` executes every stage in a single persistent kernel
(``nibble_chain_run``): each CU's compute waves keep streaming weights across
stage boundaries while a staging wave waits for the stage's inputs, so the
~3.5 us per-launch floor of the small projections is paid once per chain.

Every output has the bits of :func:`~nibblegemm_amd.ops.matmul` /
:func:`~nibblegemm_amd.ops.matmul_bias` / :func:`~nibblegemm_amd.ops.matmul_swiglu`
on the same strip-major weight: the chain runs each strip with the strip
kernel's waves, quant-group ranges, MFMA sequence and reduction order.  A
packed weight read as strips of some width gives the bits of its strip-major
copy at that width: a wave's 1 KiB load takes the strip's rows piece by piece,
so the bytes in LDS are the same.

A chain records raw pointers: its tensors are kept alive by the chain and
must not be reallocated; write new inputs into them in place.  A run
allocates nothing, so it can be captured into a HIP graph (runs of one chain
must not overlap: they share its stage counters).

    chain = DecodeChain([stage(x, w_qkv), stage(..., after=0), ...])
    chain.run()
    chain.check()   # synchronises; raises if a run gave up waiting
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import List, Optional, Sequence, Union

import torch

from . import _native
from .quant import SWIGLU_BLOCK, QuantizedWeight, StripMajorWeight

EPILOGUE_NONE, EPILOGUE_BIAS, EPILOGUE_SWIGLU = 0, 1, 2
# nibble_chain_stage: X, Wt, St, Y, bias pointers, then K, N, group_size,
# strip_cols, epilogue, after, layout (include/nibblegemm_amd.h).
_STAGE = struct.Struct("<5Q7q")
LAYOUT_STRIP_MAJOR, LAYOUT_PACKED = 0, 1


def chain_strip_cols(K: int, N: int, group_size: int, M: int = 1) -> int:
    """The strip width a chain of independent ``M``-row stages streams a
    ``[K, N]`` weight fastest at (``nibble_chain_strip_cols``): the widest of
    64 and 32 columns the chain has a plan for, else
    :func:`~nibblegemm_amd.ops.strip_major_cols`'s width; 0 when none fits a
    chain.  A chain round costs a fixed allowance besides its bytes, so a
    chain of many stages wants fewer, wider strips than the per-projection
    launches do; a weight converted at either width serves both
    (``ops.to_strip_major(qw, chain_strip_cols(...))``)."""
    return int(_native.binding().chain_strip_cols(K, N, group_size, M))


@dataclass
class Stage:
    """One stage: ``Y = epilogue(X @ W)``.  ``after`` is the index of an
    earlier stage that must finish before this one reads ``X`` and ``bias``
    (-1: none).  ``W`` is strip-major, or the packed weight of the reference's
    format read as strips of ``strip_cols`` columns (the same bits)."""

    X: torch.Tensor
    W: Union[StripMajorWeight, QuantizedWeight]
    Y: torch.Tensor
    bias: Optional[torch.Tensor] = None
    epilogue: int = EPILOGUE_NONE
    after: int = -1
    strip_cols: int = 0  # packed weights: the strips the chain reads them as

    @property
    def layout(self) -> int:
        return LAYOUT_STRIP_MAJOR if isinstance(self.W, StripMajorWeight) else LAYOUT_PACKED

    @property
    def cols(self) -> int:
        return self.W.strip_cols if isinstance(self.W, StripMajorWeight) else self.strip_cols


def stage(X: torch.Tensor, W: Union[StripMajorWeight, QuantizedWeight], *,
          bias: Optional[torch.Tensor] = None, swiglu: bool = False, after: int = -1,
          Y: Optional[torch.Tensor] = None, strip_cols: int = 0) -> Stage:
    """A :class:`Stage` with its output allocated (``[M, N]``, or ``[M, N / 2]``
    for the SwiGLU epilogue of an ``interleave_swiglu`` weight).  A packed
    ``W`` (the reference's layout, unconverted) is read as strips of
    ``strip_cols`` columns, by default :func:`chain_strip_cols`'s."""
    if bias is not None and swiglu:
        raise ValueError("bias and swiglu epilogues are exclusive")
    n_out = W.N // 2 if swiglu else W.N
    if Y is None:
        Y = torch.empty((X.shape[0], n_out), dtype=torch.float16, device=X.device)
    ep = EPILOGUE_SWIGLU if swiglu else EPILOGUE_BIAS if bias is not None else EPILOGUE_NONE
    if isinstance(W, StripMajorWeight):
        if strip_cols not in (0, W.strip_cols):
            raise ValueError(f"a strip-major weight is read as its own {W.strip_cols}-column strips")
        return Stage(X, W, Y, bias, ep, after)
    if not isinstance(W, QuantizedWeight):
        raise TypeError("the weight must be a QuantizedWeight or a StripMajorWeight")
    sw = int(strip_cols) or chain_strip_cols(W.K, W.N, W.group_size, X.shape[0])
    if sw == 0:
        raise ValueError(f"no chain plan for K={W.K}, N={W.N}, group_size={W.group_size}")
    return Stage(X, W, Y, bias, ep, after, sw)


def _check(i: int, s: Stage, M: int, device: torch.device) -> None:
    w = s.W
    if not isinstance(w, (StripMajorWeight, QuantizedWeight)):
        raise TypeError(f"stage {i}: the weight must be a QuantizedWeight or a StripMajorWeight")
    tensors = [s.X, w.qweight, w.scales, s.Y] + ([s.bias] if s.bias is not None else [])
    if any(t.device != device for t in tensors):
        raise RuntimeError(f"stage {i}: all tensors must live on {device}")
    if s.X.dtype != torch.float16 or s.Y.dtype != torch.float16 or (
            s.bias is not None and s.bias.dtype != torch.float16):
        raise RuntimeError(f"stage {i}: activations, outputs and biases must be fp16")
    if w.qweight.dtype != torch.int32 or w.scales.dtype != torch.float16:
        raise RuntimeError(f"stage {i}: weights must be int32 and scales fp16")
    if not all(t.is_contiguous() for t in tensors):
        raise RuntimeError(f"stage {i}: tensors must be contiguous")
    if s.layout == LAYOUT_PACKED and (
            tuple(w.qweight.shape) != (w.K // 8, w.N)
            or tuple(w.scales.shape) != (w.K // w.group_size, w.N)):
        raise ValueError(f"stage {i}: packed weights must be [K/8, N] words and [K/G, N] scales")
    n_out = w.N // 2 if s.epilogue == EPILOGUE_SWIGLU else w.N
    if tuple(s.X.shape) != (M, w.K):
        raise ValueError(f"stage {i}: X is {tuple(s.X.shape)}, expected ({M}, {w.K})")
    if tuple(s.Y.shape) != (M, n_out):
        raise ValueError(f"stage {i}: Y is {tuple(s.Y.shape)}, expected ({M}, {n_out})")
    if s.bias is not None and (s.bias.dim() != 1 or s.bias.numel() != w.N):
        raise ValueError(f"stage {i}: bias must be [{w.N}]")
    if s.epilogue == EPILOGUE_SWIGLU and w.N % (2 * SWIGLU_BLOCK):
        raise ValueError(f"stage {i}: N={w.N} is not an interleaved gate|up weight")


class DecodeChain:
    """A list of stages run by one persistent launch (see the module notes)."""

    def __init__(self, stages: Sequence[Stage], M: int = 1):
        if not stages:
            raise ValueError("a chain needs at least one stage")
        ext = _native.binding()
        self._ext = ext
        self.M = int(M)
        self.stages: List[Stage] = list(stages)
        self.device = self.stages[0].X.device
        if self.device.type != "cuda":
            raise RuntimeError("tensors must live on the GPU")
        packed = []
        for i, s in enumerate(self.stages):
            _check(i, s, self.M, self.device)
            w = s.W
            packed.append(_STAGE.pack(
                s.X.data_ptr(), w.qweight.data_ptr(), w.scales.data_ptr(), s.Y.data_ptr(),
                s.bias.data_ptr() if s.bias is not None else 0,
                w.K, w.N, w.group_size, s.cols, s.epilogue, int(s.after), s.layout))
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            rc, handle = ext.chain_create(b"".join(packed), len(self.stages), self.M, stream)
        if rc:
            raise RuntimeError(f"nibblegemm_amd: {ext.last_error()} (status {rc})")
        self._handle = handle

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def run(self, timestamps: Optional[torch.Tensor] = None) -> None:
        """Every stage, once, on the current stream.  ``timestamps``: an
        int64 tensor of ``len(stages) + 1`` on the chain's device, filled by
        :meth:`new_timestamps`; the run records per stage the s_memrealtime
        tick (100 MHz) at which its last round ended, and in the last entry
        the tick the first workgroup started."""
        ptr = None
        if timestamps is not None:
            if (timestamps.dtype != torch.int64 or timestamps.numel() != len(self.stages) + 1
                    or timestamps.device != self.device or not timestamps.is_contiguous()):
                raise ValueError("timestamps must be a contiguous int64 tensor of "
                                 f"{len(self.stages) + 1} on {self.device}")
            ptr = timestamps.data_ptr()
        rc = self._ext.chain_run(self._handle, ptr, self._stream())
        if rc:
            raise RuntimeError(f"nibblegemm_amd: {self._ext.last_error()} (status {rc})")

    def new_timestamps(self) -> torch.Tensor:
        t = torch.zeros(len(self.stages) + 1, dtype=torch.int64, device=self.device)
        t[-1] = -1  # all ones: the start is an unsigned minimum
        return t

    @staticmethod
    def stage_times_us(timestamps: torch.Tensor) -> List[float]:
        """Per stage, the time from the chain's start to the end of its last
        round, in microseconds."""
        t = timestamps.cpu().tolist()
        start = t[-1]
        return [(x - start) / 100.0 for x in t[:-1]]

    def check(self) -> None:
        """Synchronises the current stream and raises RuntimeError if a run
        gave up waiting for a stage (its outputs are then incomplete)."""
        rc = self._ext.chain_check(self._handle, self._stream())
        if rc:
            raise RuntimeError(f"nibblegemm_amd: {self._ext.last_error()} (status {rc})")

    @property
    def workgroups(self) -> int:
        return int(self._ext.chain_info(self._handle, 0))

    @property
    def rounds(self) -> int:
        return int(self._ext.chain_info(self._handle, 1))

    @property
    def lds_bytes(self) -> int:
        return int(self._ext.chain_info(self._handle, 2))

    def outputs(self) -> List[torch.Tensor]:
        return [s.Y for s in self.stages]

    def close(self) -> None:
        h, self._handle = getattr(self, "_handle", None), None
        if h is not None:
            self._ext.chain_destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass
