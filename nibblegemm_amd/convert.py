"""Ingestion of 4-bit checkpoints stored in the GPTQ and AWQ layouts.

Both layouts describe ``w[k, n] = (q[k, n] - z[g, n]) * s[g, n]`` with 4-bit
``q``, 4-bit zero points ``z`` and fp16 scales ``s`` per group ``g = k // G``
of rows along K -- the format of this package with one restriction: its zero
point is the implicit constant 8 (symmetric INT4, no zero-point tensor; the
reference's quant.py:8-39).  A checkpoint whose zero points are all 8 (GPTQ
and AWQ quantised with ``sym=True``) therefore converts exactly: the
nibbles are only re-ordered into this package's slot order and the scales
are kept bit for bit.  Any other zero point, or a per-row group map that is
not ``k // G`` (GPTQ act-order), cannot be represented and raises
``ValueError``.

The conversions are tensor bit operations on the input's device (CPU or
GPU) and return a :class:`~nibblegemm_amd.quant.QuantizedWeight` there.

Layouts (restated from the published packers of AutoGPTQ and AutoAWQ;
neither library is a dependency):

* GPTQ: ``qweight`` int32 ``[K/8, N]``, row ``r`` holding ``k = 8r + i`` in
  bits ``4i .. 4i+3`` (sequential order); ``qzeros`` int32 ``[K/G, N/8]``
  holding the zero point of column ``8c + i`` in bits ``4i`` of column ``c``,
  stored as ``z - 1`` by the original format (``zero_offset=1``) and as ``z``
  by the "v2" format (``zero_offset=0``); ``scales`` fp16 ``[K/G, N]``;
  optional ``g_idx`` int32 ``[K]``.
* AWQ (the "GEMM" layout): ``qweight`` int32 ``[K, N/8]`` packed along N,
  nibble ``i`` of word ``c`` holding column ``8c + AWQ_ORDER[i]``; ``qzeros``
  int32 ``[K/G, N/8]`` packed the same way; ``scales`` fp16 ``[K/G, N]``.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .quant import PACK_FACTOR, SLOT_FOR_K, ZERO_POINT, QuantizedWeight

#: AWQ's column order inside a packed word: nibble ``i`` holds column ``AWQ_ORDER[i]``.
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def _nibbles(words: torch.Tensor) -> torch.Tensor:
    """int32 ``[R, C]`` -> int64 ``[R, 8, C]``: nibble ``i`` (bits ``4i..4i+3``) of every word."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = (4 * torch.arange(PACK_FACTOR, device=words.device, dtype=torch.int64)).view(1, -1, 1)
    return (w.unsqueeze(1) >> shifts) & 0xF


def _to_int32(packed: torch.Tensor) -> torch.Tensor:
    """int64 words in ``[0, 2^32)`` -> int32 of the same bit pattern."""
    return torch.where(packed >= 1 << 31, packed - (1 << 32), packed).to(torch.int32)


def pack_interleaved(n: torch.Tensor) -> torch.Tensor:
    """``[K, N]`` integers in ``[0, 15]`` -> int32 ``[K/8, N]`` in this package's
    slot order (the layout of ``pack_nibbles``), on n's device."""
    K, N = n.shape
    if K % PACK_FACTOR:
        raise ValueError(f"K={K} must be divisible by {PACK_FACTOR}")
    blocks = n.to(torch.int64).reshape(K // PACK_FACTOR, PACK_FACTOR, N)
    packed = torch.zeros((K // PACK_FACTOR, N), dtype=torch.int64, device=n.device)
    for k_off in range(PACK_FACTOR):
        packed |= (blocks[:, k_off, :] & 0xF) << (4 * int(SLOT_FOR_K[k_off]))
    return _to_int32(packed)


def _check_scales(scales: torch.Tensor, K: int, N: int, group_size: int) -> None:
    if group_size <= 0 or group_size % PACK_FACTOR or K % group_size:
        raise ValueError(f"group_size={group_size} must divide K={K} and be a multiple of 8")
    if tuple(scales.shape) != (K // group_size, N):
        raise ValueError(f"scales must be [{K // group_size}, {N}], got {tuple(scales.shape)}")


def _require_symmetric(z: torch.Tensor, what: str) -> None:
    if bool((z != ZERO_POINT).any()):
        bad = sorted(set(int(v) for v in z.flatten().unique().tolist()) - {ZERO_POINT})
        raise ValueError(
            f"{what}: zero points other than {ZERO_POINT} ({bad[:4]}) cannot be represented; "
            f"the packed format is symmetric with an implicit zero point of {ZERO_POINT}")


def from_gptq(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int,
              g_idx: Optional[torch.Tensor] = None, zero_offset: int = 1) -> QuantizedWeight:
    """A symmetric GPTQ 4-bit checkpoint tensor set as a :class:`QuantizedWeight`."""
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise ValueError("GPTQ qweight and qzeros must be int32")
    if qweight.dim() != 2:
        raise ValueError(f"qweight must be 2-D, got {tuple(qweight.shape)}")
    K, N = qweight.shape[0] * PACK_FACTOR, qweight.shape[1]
    _check_scales(scales, K, N, group_size)
    if N % PACK_FACTOR or tuple(qzeros.shape) != (K // group_size, N // PACK_FACTOR):
        raise ValueError(f"qzeros must be [{K // group_size}, {N // PACK_FACTOR}], "
                         f"got {tuple(qzeros.shape)}")
    if g_idx is not None:
        expect = torch.arange(K, device=g_idx.device, dtype=torch.int64) // group_size
        if g_idx.numel() != K or bool((g_idx.to(torch.int64) != expect).any()):
            raise ValueError("g_idx is not k // group_size (act-order checkpoint): the packed "
                             "format needs contiguous groups along K")
    z = _nibbles(qzeros).permute(0, 2, 1).reshape(K // group_size, N) + zero_offset
    _require_symmetric(z, "GPTQ checkpoint")
    n = _nibbles(qweight).reshape(K, N)  # [r, i, c] -> row 8r + i
    return QuantizedWeight(pack_interleaved(n).contiguous(),
                           scales.to(torch.float16).contiguous(), group_size, K, N)


def to_gptq(qw: QuantizedWeight, zero_offset: int = 1
            ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The GPTQ layout of ``qw``: ``(qweight, qzeros, scales, g_idx)`` on qw's device."""
    K, N, g = qw.K, qw.N, qw.group_size
    if N % PACK_FACTOR:
        raise ValueError(f"N={N} must be divisible by {PACK_FACTOR} for GPTQ zero packing")
    dev = qw.qweight.device
    # Slot s of a word holds k = K_FOR_SLOT[s]; read nibbles back in k order.
    slots = _nibbles(qw.qweight)  # [K/8, slot, N]
    order = torch.as_tensor(SLOT_FOR_K, device=dev)
    n = slots.index_select(1, order)  # [K/8, k, N]
    shifts = (4 * torch.arange(PACK_FACTOR, device=dev, dtype=torch.int64)).view(1, -1, 1)
    qweight = _to_int32((n << shifts).sum(dim=1))
    zs = torch.full((K // g, N // PACK_FACTOR, PACK_FACTOR), ZERO_POINT - zero_offset,
                    dtype=torch.int64, device=dev)
    qzeros = _to_int32((zs << shifts.view(1, 1, -1)).sum(dim=2))
    g_idx = (torch.arange(K, device=dev, dtype=torch.int64) // g).to(torch.int32)
    return qweight.contiguous(), qzeros.contiguous(), qw.scales.clone(), g_idx


def _unpack_awq(words: torch.Tensor) -> torch.Tensor:
    """int32 ``[R, N/8]`` in AWQ column order -> int64 ``[R, N]`` in column order."""
    R, C = words.shape
    nib = _nibbles(words)  # [R, i, c]: column 8c + AWQ_ORDER[i]
    inv = [AWQ_ORDER.index(j) for j in range(PACK_FACTOR)]
    cols = nib.index_select(1, torch.as_tensor(inv, device=words.device))  # [R, j, c]
    return cols.permute(0, 2, 1).reshape(R, C * PACK_FACTOR)


def from_awq(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
             group_size: int) -> QuantizedWeight:
    """A symmetric AWQ ("GEMM" layout) 4-bit checkpoint tensor set as a
    :class:`QuantizedWeight`."""
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise ValueError("AWQ qweight and qzeros must be int32")
    if qweight.dim() != 2:
        raise ValueError(f"qweight must be 2-D, got {tuple(qweight.shape)}")
    K, N = qweight.shape[0], qweight.shape[1] * PACK_FACTOR
    _check_scales(scales, K, N, group_size)
    if tuple(qzeros.shape) != (K // group_size, N // PACK_FACTOR):
        raise ValueError(f"qzeros must be [{K // group_size}, {N // PACK_FACTOR}], "
                         f"got {tuple(qzeros.shape)}")
    _require_symmetric(_unpack_awq(qzeros), "AWQ checkpoint")
    n = _unpack_awq(qweight)
    return QuantizedWeight(pack_interleaved(n).contiguous(),
                           scales.to(torch.float16).contiguous(), group_size, K, N)
