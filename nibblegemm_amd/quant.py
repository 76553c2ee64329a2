"""Packed INT4 weight format: quantiser, packer and host-side decode.

Drop-in for ``python/nibblegemm/quant.py`` of arvindcr4/nibblegemm: same names,
same array shapes and dtypes, same errors.

Format (reference quant.py:8-54)
--------------------------------
``W`` is ``[K, N]`` and consumed as ``Y = X @ W`` (K is the reduction axis).

* Groups of ``group_size`` rows along K share one fp16 scale per column.
* Symmetric INT4: ``q = clamp(round_half_even(w / scale), -8, 7)``, stored as
  ``q + 8`` in ``[0, 15]``; there is no zero-point tensor.
* ``scale = max(max|w| / 7, 1e-8)`` per group and column (plain max-abs).
* Eight nibbles along K share one 32-bit word: ``qweight`` is int32
  ``[K // 8, N]``.  Logical offset ``k`` of a word lives in nibble slot
  ``SLOT_FOR_K[k] = [0, 4, 1, 5, 2, 6, 3, 7]`` (even k in slots 0..3, odd k in
  slots 4..7), the order in which the kernels' mask-and-or decode emits fp16
  pairs in ascending k.

Host code only: packing happens at quantisation time, ``dequantize`` and
``reference_matmul`` reproduce the reference's definitions for callers' own
checks.  The kernel entry points in :mod:`nibblegemm_amd.ops` never call them.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

#: ``SLOT_FOR_K[k]`` is the nibble slot that stores logical offset ``k`` (0..7).
SLOT_FOR_K = np.array([0, 4, 1, 5, 2, 6, 3, 7], dtype=np.int64)
#: Inverse permutation: ``K_FOR_SLOT[s]`` is the logical offset held by slot ``s``.
K_FOR_SLOT = np.argsort(SLOT_FOR_K)

QMIN, QMAX = -8, 7
ZERO_POINT = 8
PACK_FACTOR = 8


@dataclass(frozen=True)
class QuantizedWeight:
    """Packed INT4 weights plus their fp16 group scales (reference quant.py:60-78)."""

    qweight: torch.Tensor  # int32 [K // 8, N], nibble-interleaved
    scales: torch.Tensor  # fp16  [K // G, N]
    group_size: int
    K: int
    N: int

    def to(self, device) -> "QuantizedWeight":
        return QuantizedWeight(
            self.qweight.to(device), self.scales.to(device), self.group_size, self.K, self.N
        )

    @property
    def weight_bytes(self) -> int:
        """Bytes of weight traffic a perfect kernel must read (packed + scales)."""
        return self.qweight.numel() * 4 + self.scales.numel() * 2


# Clipping ratios the scale search tries, largest first (reference quant.py:57).
CLIP_RATIOS = torch.linspace(1.0, 0.55, 19)


def _search_scale(groups: torch.Tensor, n_chunk: int = 4096) -> torch.Tensor:
    """Per-group scale minimising the group's squared quantisation error over
    the clipping ratios ``CLIP_RATIOS`` (reference quant.py:81-124): for each
    ratio r, ``scale = max(amax * r / 7, 1e-8)``, the group rounded with it,
    and the sum of squared errors; a later ratio replaces the best so far only
    when strictly better.  The reference keeps it as a documented negative
    result (lower weight error, worse model quality); it is off by default.

    groups: float32 ``[K/G, G, N]`` -> scales ``[K/G, N]``, on groups' device,
    processed ``n_chunk`` columns at a time."""
    n_groups, _, N = groups.shape
    out = torch.empty((n_groups, N), dtype=groups.dtype, device=groups.device)
    ratios = CLIP_RATIOS.to(groups.device, groups.dtype)
    for c0 in range(0, N, n_chunk):
        blk = groups[:, :, c0:c0 + n_chunk]
        amax = blk.abs().amax(dim=1)
        best = (amax / QMAX).clamp(min=1e-8)
        best_err = torch.full_like(amax, float("inf"))
        for r in ratios:
            s = (amax * r / QMAX).clamp(min=1e-8)
            q = torch.round(blk / s.unsqueeze(1)).clamp(QMIN, QMAX)
            err = (q * s.unsqueeze(1) - blk).pow(2).sum(dim=1)
            take = err < best_err
            best_err = torch.where(take, err, best_err)
            best = torch.where(take, s, best)
        out[:, c0:c0 + n_chunk] = best
    return out


def quantize(W: torch.Tensor, group_size: int = 128, clip_search: bool = False) -> QuantizedWeight:
    """Round-to-nearest quantise a ``[K, N]`` weight to packed group-wise INT4.

    Reference quant.py:127-161.  ``clip_search`` picks each group's scale by
    :func:`_search_scale` instead of max-abs (off by default, as in the
    reference, which documents it as lowering model quality).  The work runs
    on W's device; the result is on the host.
    """
    if W.ndim != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(W.shape)}")
    K, N = W.shape
    if K % group_size:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    if group_size % PACK_FACTOR:
        raise ValueError(f"group_size={group_size} must be divisible by {PACK_FACTOR}")

    w = W.detach().float()
    groups = w.reshape(K // group_size, group_size, N)
    if clip_search:
        scale = _search_scale(groups)
    else:
        # Clamp away exact zeros so all-zero groups stay finite.
        scale = (groups.abs().amax(dim=1) / QMAX).clamp(min=1e-8)
    q = torch.round(groups / scale.unsqueeze(1)).clamp(QMIN, QMAX)
    qu = (q + ZERO_POINT).reshape(K, N).to(torch.uint8).cpu().numpy()

    return QuantizedWeight(
        qweight=torch.from_numpy(pack_nibbles(qu)),
        scales=scale.to(torch.float16).cpu().contiguous(),
        group_size=group_size,
        K=K,
        N=N,
    )


def quantize_device(W: torch.Tensor, group_size: int = 128) -> QuantizedWeight:
    """:func:`quantize` without leaving W's device: the same round-to-nearest
    INT4 and the same packed layout, bit for bit, with ``qweight`` and
    ``scales`` on W's device.  For building large weight stacks on the GPU
    (the reference's ``quantize`` always returns host tensors,
    python/nibblegemm/quant.py:154-161).
    """
    if W.ndim != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(W.shape)}")
    K, N = W.shape
    if K % group_size:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    if group_size % PACK_FACTOR:
        raise ValueError(f"group_size={group_size} must be divisible by {PACK_FACTOR}")

    groups = W.detach().float().reshape(K // group_size, group_size, N)
    amax = groups.abs().amax(dim=1)
    # A tensor divisor, not the Python scalar 7: on the GPU a scalar divisor is
    # applied as a multiply by its reciprocal, which can round differently
    # from the true division the host path performs.
    scale = (amax / torch.full_like(amax, float(QMAX))).clamp(min=1e-8)
    q = torch.round(groups / scale.unsqueeze(1)).clamp(QMIN, QMAX)
    packed = pack_nibbles_device((q + ZERO_POINT).reshape(K, N))
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


#: Column block of :func:`interleave_swiglu` (half of the kernels' 64-column strip).
SWIGLU_BLOCK = 32


def interleave_swiglu(gate: QuantizedWeight, up: QuantizedWeight) -> QuantizedWeight:
    """The gate and up projections of a SwiGLU MLP as one ``[K, 2N]`` weight
    whose columns alternate in blocks of 32: gate 0..31, up 0..31, gate
    32..63, ...  Every 64-column strip of the kernels then holds matching
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


def pack_nibbles(qu: np.ndarray) -> np.ndarray:
    """Pack ``uint8 [K, N]`` values in ``[0, 15]`` into ``int32 [K // 8, N]``.

    Works in uint32 so the top nibble cannot trip signed overflow, then views
    the result as int32 (the dtype the kernels take).  Reference quant.py:164-182.
    """
    qu = np.asarray(qu)
    K, N = qu.shape
    if K % PACK_FACTOR:
        raise ValueError(f"K={K} must be divisible by {PACK_FACTOR}")
    if qu.max(initial=0) > 15:
        raise ValueError("quantised values must fit in 4 bits")

    blocks = qu.reshape(K // PACK_FACTOR, PACK_FACTOR, N).astype(np.uint32)
    packed = np.zeros((K // PACK_FACTOR, N), dtype=np.uint32)
    for k_off in range(PACK_FACTOR):
        packed |= (blocks[:, k_off, :] & np.uint32(0xF)) << np.uint32(4 * int(SLOT_FOR_K[k_off]))
    return packed.view(np.int32)


def unpack_nibbles(packed: np.ndarray, K: int) -> np.ndarray:
    """Inverse of :func:`pack_nibbles`; returns ``uint8 [K, N]`` in ``[0, 15]``
    (reference quant.py:185-196)."""
    p = np.ascontiguousarray(packed).view(np.uint32)
    rows, N = p.shape
    if rows * PACK_FACTOR != K:
        raise ValueError(f"packed rows={rows} inconsistent with K={K}")
    out = np.empty((rows, PACK_FACTOR, N), dtype=np.uint8)
    for k_off in range(PACK_FACTOR):
        out[:, k_off, :] = ((p >> np.uint32(4 * int(SLOT_FOR_K[k_off]))) & np.uint32(0xF)).astype(np.uint8)
    return out.reshape(K, N)


def dequantize(qw: QuantizedWeight) -> torch.Tensor:
    """The ``[K, N]`` fp16 weight the kernels model, on the host:
    ``fp16((nibble - 8) * fp32(scale))`` (reference quant.py:199-204).
    The device kernel for the same result is :func:`nibblegemm_amd.ops.dequant`."""
    qu = unpack_nibbles(qw.qweight.cpu().numpy(), qw.K)
    q = torch.from_numpy(qu.astype(np.int16)).float() - ZERO_POINT
    scale = qw.scales.float().cpu().repeat_interleave(qw.group_size, dim=0)
    return (q * scale).to(torch.float16)


def reference_matmul(X: torch.Tensor, qw: QuantizedWeight) -> torch.Tensor:
    """fp32-accumulated ``X @ dequantize(qw)`` rounded to fp16, on X's device
    (reference quant.py:207-215)."""
    W = dequantize(qw).to(X.device).float()
    return (X.float() @ W).to(torch.float16)
