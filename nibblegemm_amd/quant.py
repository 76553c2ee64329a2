"""The packed INT4 weight format and its host-side tools.

Drop-in for ``python/nibblegemm/quant.py`` of arvindcr4/nibblegemm: the public
names, argument orders, dtypes and exceptions are that module's (callers and
checkpoints move over unchanged); the code is this package's own.

Layout (the reference documents it at quant.py:8-54)
----------------------------------------------------
A weight ``W`` is ``[K, N]`` and is applied as ``Y = X @ W``.  Every run of
``group_size`` consecutive k shares one fp16 scale per column (``scales`` is
``[K / group_size, N]``).  A weight is stored as the 4-bit code
``round_half_even(w / scale)`` clamped to ``[-8, 7]`` and offset by 8, so codes
are ``0..15`` and the zero point is implicit.  The scale of a group column is
its largest magnitude divided by 7 (never below 1e-8).

Codes are packed eight to a 32-bit word along K (``qweight`` is int32
``[K / 8, N]``).  Code k of a word occupies bits ``4 * SLOT_FOR_K[k]`` up: the
even k take the low four nibbles and the odd k the high four, which is what
lets the kernels turn two codes sixteen bits apart into one fp16 pair with a
single mask-and-or.

This module never launches a kernel; :mod:`nibblegemm_amd.ops` never calls its
host decoders.
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass

import numpy as np
import torch

#: Nibble slot of each logical k within a packed word.
SLOT_FOR_K = np.array([0, 4, 1, 5, 2, 6, 3, 7], dtype=np.int64)
#: Logical k held by each nibble slot (the inverse permutation).
K_FOR_SLOT = np.argsort(SLOT_FOR_K)

QMIN, QMAX = -8, 7
ZERO_POINT = 8
PACK_FACTOR = 8

_SHIFTS = (4 * SLOT_FOR_K).astype(np.uint32)  # bit offset of each k's nibble


@dataclass(frozen=True)
class QuantizedWeight:
    """One quantised ``[K, N]`` weight: the packed codes, the group scales and
    the shape they describe (reference quant.py:60-78)."""

    qweight: torch.Tensor  # int32 [K // 8, N]
    scales: torch.Tensor  # fp16  [K // group_size, N]
    group_size: int
    K: int
    N: int

    def to(self, device) -> "QuantizedWeight":
        """The same weight with both tensors moved to ``device``."""
        return dataclasses.replace(self, qweight=self.qweight.to(device),
                                   scales=self.scales.to(device))

    @property
    def weight_bytes(self) -> int:
        """Bytes a matmul must read for this weight: packed codes and scales."""
        return sum(t.numel() * t.element_size() for t in (self.qweight, self.scales))


#: Clip ratios of the optional scale search, from 1.0 (plain max-abs) down.
CLIP_RATIOS = torch.linspace(1.0, 0.55, 19)


def _check_quantize_args(W: torch.Tensor, group_size: int):
    if W.ndim != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(W.shape)}")
    K, N = W.shape
    if K % group_size:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    if group_size % PACK_FACTOR:
        raise ValueError(f"group_size={group_size} must be divisible by {PACK_FACTOR}")
    return K, N


def _codes(groups: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Offset 4-bit codes (0..15, float) of ``groups`` ``[K/G, G, N]`` at the
    per-group-column ``scale`` ``[K/G, N]``: half-even rounding of the true
    quotient, clamped to the signed range, plus the zero point."""
    return torch.round(groups / scale[:, None, :]).clamp(QMIN, QMAX) + ZERO_POINT


def _search_scale(groups: torch.Tensor, n_chunk: int = 4096) -> torch.Tensor:
    """Scales chosen by squared quantisation error instead of max-abs
    (reference quant.py:81-124, which keeps it, off by default, as a measured
    negative result for model quality).

    Each candidate is ``max(amax * r / 7, 1e-8)`` for the ratios r of
    ``CLIP_RATIOS``; the error of a group column is the sum over the group of
    ``(q * s - w)^2`` in float32.  The pick is the first candidate reaching the
    smallest error, so ratio 1.0 (max-abs) wins every tie.  ``groups`` is
    float32 ``[K/G, G, N]``; the result ``[K/G, N]`` is on its device, worked
    out ``n_chunk`` columns at a time."""
    n_groups, _, N = groups.shape
    ratios = CLIP_RATIOS.to(groups.device, groups.dtype)
    out = torch.empty((n_groups, N), dtype=groups.dtype, device=groups.device)
    for lo in range(0, N, n_chunk):
        w = groups[:, :, lo:lo + n_chunk]
        amax = w.abs().amax(dim=1)
        cands = []
        errs = []
        for r in ratios:
            s = (amax * r / QMAX).clamp(min=1e-8)
            q = torch.round(w / s[:, None, :]).clamp(QMIN, QMAX)
            errs.append((q * s[:, None, :] - w).pow(2).sum(dim=1))
            cands.append(s)
        pick = torch.stack(errs).argmin(dim=0, keepdim=True)  # first minimum
        out[:, lo:lo + n_chunk] = torch.stack(cands).gather(0, pick)[0]
    return out


def quantize(W: torch.Tensor, group_size: int = 128, clip_search: bool = False) -> QuantizedWeight:
    """Round-to-nearest group-wise INT4 of a ``[K, N]`` weight (reference
    quant.py:127-161).  The arithmetic runs on W's device, in float32, with the
    reference's operations (the max-abs scale divides by the Python scalar 7);
    the packed result is returned on the host.  ``clip_search`` takes the
    scales from :func:`_search_scale` instead."""
    K, N = _check_quantize_args(W, group_size)
    groups = W.detach().float().reshape(K // group_size, group_size, N)
    if clip_search:
        scale = _search_scale(groups)
    else:
        scale = (groups.abs().amax(dim=1) / QMAX).clamp(min=1e-8)  # all-zero groups stay finite
    codes = _codes(groups, scale).reshape(K, N).to(torch.uint8).cpu().numpy()
    return QuantizedWeight(torch.from_numpy(pack_nibbles(codes)),
                           scale.to(torch.float16).cpu().contiguous(), group_size, K, N)


def quantize_device(W: torch.Tensor, group_size: int = 128) -> QuantizedWeight:
    """:func:`quantize` kept on W's device: the same codes, scales and packed
    layout, with ``qweight`` and ``scales`` left where W is (for building large
    weight stacks on the GPU; the reference's ``quantize`` always returns host
    tensors).  The max-abs scale divides by a tensor of 7s: a GPU divides by a
    Python scalar as a multiply by its reciprocal, which can round differently
    from the true division a host ``quantize`` performs."""
    K, N = _check_quantize_args(W, group_size)
    groups = W.detach().float().reshape(K // group_size, group_size, N)
    amax = groups.abs().amax(dim=1)
    scale = (amax / torch.full_like(amax, float(QMAX))).clamp(min=1e-8)
    packed = pack_nibbles_device(_codes(groups, scale).reshape(K, N))
    return QuantizedWeight(packed, scale.to(torch.float16).contiguous(), group_size, K, N)


def pack_nibbles_device(qu: torch.Tensor) -> torch.Tensor:
    """:func:`pack_nibbles` on a torch tensor, on its device: [K, N] values in
    [0, 15] (any integer or float dtype holding integers) -> int32 [K/8, N]."""
    K, N = qu.shape
    if K % PACK_FACTOR:
        raise ValueError(f"K={K} must be divisible by {PACK_FACTOR}")
    q = qu.to(torch.int64).reshape(K // PACK_FACTOR, PACK_FACTOR, N)
    packed = torch.zeros((K // PACK_FACTOR, N), dtype=torch.int64, device=qu.device)
    for k_off in range(PACK_FACTOR):
        packed |= q[:, k_off, :] << (4 * int(SLOT_FOR_K[k_off]))
    # Words with the top bit set are the negative int32 of the same bit pattern.
    return torch.where(packed >= 1 << 31, packed - (1 << 32), packed).to(torch.int32).contiguous()


def concat_columns(*qws: QuantizedWeight) -> QuantizedWeight:
    """Weights that share K and the group size, side by side as one ``[K, sum N]``
    weight.  Packing runs along K, so concatenating packed columns and scale
    columns gives exactly the packed form of the concatenated dense weights;
    ``X @ concat(W1, W2)`` is ``[X @ W1, X @ W2]`` in one launch (e.g. the q, k
    and v projections of an attention block, or gate and up of an MLP)."""
    if not qws:
        raise ValueError("nothing to concatenate")
    K, g = qws[0].K, qws[0].group_size
    for qw in qws:
        if qw.K != K or qw.group_size != g:
            raise ValueError("concatenated weights must share K and group_size")
    return QuantizedWeight(torch.cat([qw.qweight for qw in qws], dim=1).contiguous(),
                           torch.cat([qw.scales for qw in qws], dim=1).contiguous(),
                           g, K, sum(qw.N for qw in qws))


#: Column block of :func:`interleave_swiglu`: every 32-column strip of the
#: kernels holds 16 gate columns and the matching 16 up columns.
SWIGLU_BLOCK = 16


def interleave_swiglu(gate: QuantizedWeight, up: QuantizedWeight) -> QuantizedWeight:
    """The gate and up projections of a SwiGLU MLP as one ``[K, 2N]`` weight
    whose columns alternate in blocks of 16: gate 0..15, up 0..15, gate
    16..31, ...  Every 32- or 64-column strip of the kernels then holds matching
    gate and up columns, which lets one launch write ``silu(X Wg) * (X Wu)``
    (``ops.matmul_swiglu``).  Packing runs along K, so permuting packed and
    scale columns is exact."""
    if gate.K != up.K or gate.group_size != up.group_size or gate.N != up.N:
        raise ValueError("gate and up must share K, N and group_size")
    if gate.N % SWIGLU_BLOCK:
        raise ValueError(f"N={gate.N} must be a multiple of {SWIGLU_BLOCK}")

    def mix(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        rows, n = a.shape
        blocks = n // SWIGLU_BLOCK
        return torch.stack([a.reshape(rows, blocks, SWIGLU_BLOCK),
                            b.reshape(rows, blocks, SWIGLU_BLOCK)], dim=2).reshape(rows, 2 * n)

    return QuantizedWeight(mix(gate.qweight, up.qweight).contiguous(),
                           mix(gate.scales, up.scales).contiguous(),
                           gate.group_size, gate.K, 2 * gate.N)


def split_swiglu(y: torch.Tensor):
    """Inverse column order of :func:`interleave_swiglu` on a ``[M, 2N]``
    output: returns the gate and up halves, each ``[M, N]``."""
    rows, n2 = y.shape
    blocks = n2 // (2 * SWIGLU_BLOCK)
    v = y.reshape(rows, blocks, 2, SWIGLU_BLOCK)
    return (v[:, :, 0, :].reshape(rows, n2 // 2), v[:, :, 1, :].reshape(rows, n2 // 2))


#: Strip widths of the strip-major layout (columns per strip).
STRIP_COLS = (16, 32, 64)


@dataclass(frozen=True)
class StripMajorWeight:
    """A quantised ``[K, N]`` weight in the strip-major layout of the decode
    GEMV (an MI355X layout; the reference has only the packed one).  The N
    columns are cut into strips of ``strip_cols`` and each strip is stored
    whole: ``qweight`` int32 ``[N / strip_cols, K / 8, strip_cols]`` and
    ``scales`` fp16 ``[N / strip_cols, K / group_size, strip_cols]`` hold the
    words and scales of the packed layout, permuted (:func:`strip_major`).  A
    decode workgroup then reads one contiguous run per strip.  Serves every
    batch size (:func:`nibblegemm_amd.ops.to_strip_major` makes one on the
    device; :func:`from_strip_major` restores the packed weight)."""

    qweight: torch.Tensor
    scales: torch.Tensor
    group_size: int
    K: int
    N: int
    strip_cols: int

    def to(self, device) -> "StripMajorWeight":
        return dataclasses.replace(self, qweight=self.qweight.to(device),
                                   scales=self.scales.to(device))

    @property
    def weight_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.qweight, self.scales))


def strip_major(qw: QuantizedWeight, strip_cols: int) -> StripMajorWeight:
    """The strip-major copy of ``qw`` by tensor reshapes on its own device
    (the layout's definition: word ``[s][r][j]`` is packed word ``[r][s *
    strip_cols + j]``, scale ``[s][g][j]`` is scale ``[g][s * strip_cols +
    j]``)."""
    if strip_cols not in STRIP_COLS:
        raise ValueError(f"strip_cols must be one of {STRIP_COLS}, got {strip_cols}")
    if qw.N % strip_cols:
        raise ValueError(f"N={qw.N} is not a multiple of strip_cols={strip_cols}")

    def cut(t: torch.Tensor) -> torch.Tensor:
        rows, n = t.shape
        return t.reshape(rows, n // strip_cols, strip_cols).permute(1, 0, 2).contiguous()

    return StripMajorWeight(cut(qw.qweight), cut(qw.scales), qw.group_size, qw.K, qw.N, strip_cols)


def from_strip_major(sm: StripMajorWeight) -> QuantizedWeight:
    """The packed weight a strip-major one was made from (the inverse
    permutation of :func:`strip_major`, on its own device)."""

    def join(t: torch.Tensor) -> torch.Tensor:
        strips, rows, sw = t.shape
        return t.permute(1, 0, 2).reshape(rows, strips * sw).contiguous()

    return QuantizedWeight(join(sm.qweight), join(sm.scales), sm.group_size, sm.K, sm.N)


def pack_nibbles(qu: np.ndarray) -> np.ndarray:
    """Codes ``[K, N]`` (values 0..15) to packed words ``int32 [K // 8, N]``
    (reference quant.py:164-182).  Each code is masked to its low four bits
    (as the reference does, so a negative signed code wraps into its own
    nibble: -1 packs as 15), shifted to its nibble slot, and the eight of a
    word are OR-ed in uint32 (no sign to overflow into); the words are
    returned viewed as int32, the dtype the kernels take."""
    qu = np.asarray(qu)
    K, N = qu.shape
    if K % PACK_FACTOR:
        raise ValueError(f"K={K} must be divisible by {PACK_FACTOR}")
    if qu.max(initial=0) > 15:
        raise ValueError("quantised values must fit in 4 bits")
    codes = qu.reshape(K // PACK_FACTOR, PACK_FACTOR, N).astype(np.uint32) & np.uint32(0xF)
    words = np.bitwise_or.reduce(codes << _SHIFTS[None, :, None], axis=1)
    return np.ascontiguousarray(words, dtype=np.uint32).view(np.int32)


def unpack_nibbles(packed: np.ndarray, K: int) -> np.ndarray:
    """Packed words ``[K // 8, N]`` back to codes ``uint8 [K, N]`` (reference
    quant.py:185-196)."""
    words = np.ascontiguousarray(packed).view(np.uint32)
    rows, N = words.shape
    if rows * PACK_FACTOR != K:
        raise ValueError(f"packed rows={rows} inconsistent with K={K}")
    codes = (words[:, None, :] >> _SHIFTS[None, :, None]) & np.uint32(0xF)
    return codes.astype(np.uint8).reshape(K, N)


def dequantize(qw: QuantizedWeight) -> torch.Tensor:
    """The fp16 ``[K, N]`` weight a packed weight stands for, on the host
    (reference quant.py:199-204): ``(code - 8) * scale`` formed in float32 --
    exact, since both factors fit in 11 bits -- and rounded once to fp16.  The
    device kernel for the same bits is :func:`nibblegemm_amd.ops.dequant`."""
    codes = unpack_nibbles(qw.qweight.cpu().numpy(), qw.K)
    signed = codes.astype(np.float32) - np.float32(ZERO_POINT)
    per_row = np.repeat(qw.scales.cpu().numpy().astype(np.float32), qw.group_size, axis=0)
    with np.errstate(over="ignore"):  # products beyond fp16 range round to inf, as in torch
        return torch.from_numpy((signed * per_row).astype(np.float16))


def reference_matmul(X: torch.Tensor, qw: QuantizedWeight) -> torch.Tensor:
    """``X @ dequantize(qw)`` accumulated in float32 and rounded to fp16, on
    X's device (reference quant.py:207-215): the yardstick the kernels are
    tested against."""
    W = dequantize(qw).to(device=X.device, dtype=torch.float32)
    return torch.matmul(X.to(torch.float32), W).to(torch.float16)
