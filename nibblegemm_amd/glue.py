"""Decode-step glue around the W4A16 projections: RMSNorm and grouped-query
attention over a KV cache, as HIP kernels (``nibble_rmsnorm_f16`` and
``nibble_attention_decode_f16`` of the C ABI).

The reference runs these as PyTorch / transformers ops of the model it
decodes with QuantLinear layers swapped in (bench/bench_model.py:131-154,
:177-188).  Here they let a whole Llama-shaped token step -- norms,
projections, attention, residual adds -- run as kernels in one HIP graph
(:class:`nibblegemm_amd.decode_step.GlueDecodeStep`).

Like every kernel entry point of this package, these raise RuntimeError when
the native library is missing; there is no PyTorch fallback.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native
from .ops import _raise, _stream, _workspace, _ws_plan

HEAD_DIM = 128
LLAMA3_ROPE_THETA = 500000.0


def _check_f16(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must live on the GPU")
    if t.dtype != torch.float16:
        raise RuntimeError(f"{name} must be fp16, got {t.dtype}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """``fp16(x * r * weight)`` per row, ``r = 1 / sqrt(mean(x^2) + eps)``,
    computed in fp32 with one rounding (transformers' LlamaRMSNorm rounds
    ``x * r`` to fp16 before the weight).  x fp16 [rows, cols], weight fp16
    [cols]; cols a multiple of 8 up to 16384."""
    _check_f16("x", x)
    _check_f16("weight", weight)
    if x.dim() != 2 or weight.dim() != 1 or weight.numel() != x.size(1):
        raise ValueError(f"expected x [rows, cols] and weight [cols], got {tuple(x.shape)} and "
                         f"{tuple(weight.shape)}")
    if weight.device != x.device:
        raise RuntimeError("x and weight must be on the same device")
    ext = _native.binding()
    y = torch.empty_like(x)
    rc = ext.rmsnorm(x.data_ptr(), x.size(0), x.size(1), weight.data_ptr(), float(eps),
                     y.data_ptr(), _stream(x.device))
    if rc:
        _raise(rc, ext)
    return y


def rope_tables(max_seq: int, head_dim: int = HEAD_DIM, theta: float = LLAMA3_ROPE_THETA,
                device="cuda") -> Tuple[torch.Tensor, torch.Tensor]:
    """cos and sin, fp32 [max_seq, head_dim / 2], of the rotary embedding
    ``angle(p, i) = p * theta^(-2 i / head_dim)`` (computed in float64)."""
    inv = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim)
    ang = torch.outer(torch.arange(max_seq, dtype=torch.float64), inv)
    return (ang.cos().float().to(device).contiguous(), ang.sin().float().to(device).contiguous())


def attention_decode(qkv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: int,
                     rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> torch.Tensor:
    """Attention of the token at position ``pos`` over the cache, which
    holds tokens ``0 .. pos - 1``.

    qkv fp16 [1, (n_heads + 2 n_kv) * 128]: the token's q | k | v (the q|k|v
    projection's output).  k_cache, v_cache fp16 [n_kv, max_seq, 128]; the
    call writes the token's k (rotated) and v at row ``pos``.  Returns fp16
    [1, n_heads * 128] = ``softmax(q k^T / sqrt(128)) v`` per query head,
    head i reading kv head ``i // (n_heads // n_kv)``.  ``rope`` is the
    (cos, sin) pair of :func:`rope_tables` or None."""
    for name, t in (("qkv", qkv), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check_f16(name, t)
    if k_cache.dim() != 3 or k_cache.shape != v_cache.shape or k_cache.size(2) != HEAD_DIM:
        raise ValueError(f"caches must both be [n_kv, max_seq, {HEAD_DIM}], got "
                         f"{tuple(k_cache.shape)} and {tuple(v_cache.shape)}")
    n_kv, max_seq = k_cache.size(0), k_cache.size(1)
    if qkv.dim() != 2 or qkv.size(0) != 1 or qkv.size(1) % HEAD_DIM:
        raise ValueError(f"qkv must be [1, (n_heads + 2 n_kv) * {HEAD_DIM}], got {tuple(qkv.shape)}")
    n_heads = qkv.size(1) // HEAD_DIM - 2 * n_kv
    if rope is not None:
        cos, sin = rope
        for name, t in (("rope cos", cos), ("rope sin", sin)):
            if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
                raise RuntimeError(f"{name} must be a contiguous fp32 GPU tensor")
            if t.shape != (max_seq, HEAD_DIM // 2):
                raise ValueError(f"{name} must be [{max_seq}, {HEAD_DIM // 2}], got {tuple(t.shape)}")
        cos_p, sin_p = cos.data_ptr(), sin.data_ptr()
    else:
        cos_p = sin_p = None
    ext = _native.binding()
    dev = qkv.device
    stream = _stream(dev)
    key = ("attention", n_heads, n_kv, max_seq, pos)
    plan = _ws_plan.get(key)
    if plan is None:
        plan = ext.attention_workspace_bytes(n_heads, n_kv, HEAD_DIM, max_seq, pos, stream)
        _ws_plan[key] = plan
    ws, ws_bytes = _workspace(plan, dev, stream)
    out = torch.empty((1, max(n_heads, 0) * HEAD_DIM), dtype=torch.float16, device=dev)
    rc = ext.attention(qkv.data_ptr(), n_heads, n_kv, HEAD_DIM, k_cache.data_ptr(),
                       v_cache.data_ptr(), max_seq, int(pos), cos_p, sin_p, out.data_ptr(),
                       ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    if rc:
        _raise(rc, ext)
    return out


def attention_bytes(n_kv: int, pos: int) -> int:
    """Cache bytes one call reads and writes: k and v rows 0 .. pos."""
    return 2 * n_kv * (pos + 1) * HEAD_DIM * 2


__all__ = ["HEAD_DIM", "LLAMA3_ROPE_THETA", "rmsnorm", "rope_tables", "attention_decode",
           "attention_bytes"]
