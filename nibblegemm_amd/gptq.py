"""GPTQ: error-compensated INT4 quantisation into this package's packed format.

The reference's offline quantiser (python/nibblegemm/gptq.py), after Frantar
et al., "GPTQ: Accurate Post-Training Quantization for Generative Pre-trained
Transformers" (2023).  Input channels are quantised in order; after each one,
its rounding error is pushed onto the channels not yet quantised, weighted by
the upper Cholesky factor of the inverse Hessian ``H = 2 X^T X`` of the layer's
calibration activations.  The output is the same packed layout as
:func:`~nibblegemm_amd.quant.quantize` -- only the chosen values differ -- so
every kernel consumes it unchanged.

Where the work runs: the per-channel loop of each quantisation group is one
HIP launch (``nibble_gptq_group_f32``: a thread per output row, the group's
factor in LDS), instead of one small elementwise launch per channel; the
update of the later channels after each group is a GEMM (hipBLASLt through
torch), and the factorisation is torch.linalg.  Both follow the reference's
operations in order, so on the same device the results are the reference's.
GPU only: there is no CPU path.
"""
from __future__ import annotations

from typing import Callable, Dict, Iterable, List, Optional, Tuple

import torch
import torch.nn as nn

from . import _native
from .ops import QuantLinear, _raise, _stream
from .quant import QuantizedWeight, pack_nibbles_device

__all__ = ["HessianAccumulator", "gptq_quantize", "find_decoder_blocks", "supported_linear",
           "quantize_model_gptq"]


class HessianAccumulator:
    """``H = 2 X^T X / n`` over every activation row seen so far, kept as a
    running mean (reference gptq.py:44-62), so that the damping term -- a
    fraction of ``mean(diag(H))`` -- does not depend on the token count."""

    def __init__(self, in_features: int, device, dtype=torch.float32):
        self.H = torch.zeros(in_features, in_features, device=device, dtype=dtype)
        self.n = 0

    @torch.no_grad()
    def add(self, x: torch.Tensor) -> None:
        """Folds a batch of activations ``[..., in_features]`` into H."""
        x = x.reshape(-1, x.shape[-1]).to(self.H.dtype)
        rows = x.shape[0]
        if rows == 0:
            return
        # H_new = H_old * n / (n + rows) + 2 / (n + rows) * x^T x
        self.H *= self.n / (self.n + rows)
        self.n += rows
        self.H += (2.0 / self.n) * (x.t() @ x)


def _inverse_cholesky(H: torch.Tensor, damp: float, retries: int) -> torch.Tensor:
    """Upper-triangular factor U of ``(H + lambda I)^-1 = U^T U``, the form the
    column loop reads (row i, from the diagonal on, spreads channel i's error).
    ``lambda`` starts at ``damp * mean(diag(H))`` and grows tenfold per failed
    factorisation, ``retries`` times (reference gptq.py:137-172)."""
    K = H.shape[0]
    eye = torch.eye(K, device=H.device, dtype=H.dtype)
    mean_diag = torch.diag(H).mean().clamp(min=1e-8)
    for attempt in range(retries):
        lam = damp * (10 ** attempt)
        try:
            L = torch.linalg.cholesky(H + eye * (lam * mean_diag))
            inv = torch.cholesky_inverse(L)
            # potrf fills only the requested triangle; triu makes the rest zero.
            return torch.triu(torch.linalg.cholesky(inv, upper=True))
        except RuntimeError:  # torch.linalg.LinAlgError is a RuntimeError
            continue
    raise RuntimeError(
        f"Hessian factorisation failed after {retries} attempts up to damping "
        f"{damp * 10 ** (retries - 1):.3g}; the calibration set is probably degenerate")


@torch.no_grad()
def gptq_quantize(W: torch.Tensor, H: torch.Tensor, group_size: int = 128,
                  damp: float = 0.01, max_damp_retries: int = 5) -> QuantizedWeight:
    """Quantises ``W`` ``[K, N]`` (consumed as ``Y = X @ W``) given the Hessian
    ``H`` ``[K, K]`` of its input activations (reference gptq.py:65-134).

    Groups of ``group_size`` input channels are processed in order.  A group's
    scales come from its weights *after* the compensation pushed onto them by
    the groups before it; within the group the channels are rounded one at a
    time, each error spread over the group's later channels; then the group's
    errors are spread over all later channels at once.  Channels whose
    Hessian diagonal is zero (never activated) are zeroed.

    Returns host tensors, as the reference's quantisers do.
    """
    K, N = W.shape
    if K % group_size:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    if H.shape != (K, K):
        raise ValueError(f"H must be [{K}, {K}], got {tuple(H.shape)}")
    if group_size not in (64, 128):
        raise ValueError(f"group_size must be 64 or 128, got {group_size}")
    dev = W.device if W.is_cuda else (H.device if H.is_cuda else None)
    if dev is None:
        if not torch.cuda.is_available():
            raise RuntimeError("gptq_quantize runs its column loop on the GPU; none is visible")
        dev = torch.device("cuda", torch.cuda.current_device())
    G = group_size

    # [out, in]: a row per output channel, the orientation the loop runs in.
    Wt = W.detach().to(dev).t().contiguous().float()
    H = H.detach().to(dev).float().clone()
    dead = torch.diag(H) == 0
    if dead.any():
        H[dead, dead] = 1.0
        Wt[:, dead] = 0.0
    U = _inverse_cholesky(H, damp, max_damp_retries).contiguous()

    ext = _native.binding()
    stream = _stream(dev)
    Q = torch.empty((N, K), dtype=torch.uint8, device=dev)
    scales = torch.empty((K // G, N), dtype=torch.float32, device=dev)
    E = torch.empty((N, G), dtype=torch.float32, device=dev)
    fsz = Wt.element_size()
    for i1 in range(0, K, G):
        i2 = i1 + G
        rc = ext.gptq_group(Wt.data_ptr() + i1 * fsz, K, N, G, U.data_ptr() + (i1 * K + i1) * fsz,
                            K, Q.data_ptr() + i1, K, E.data_ptr(), scales[i1 // G].data_ptr(),
                            stream)
        if rc:
            _raise(rc, ext)
        if i2 < K:
            Wt[:, i2:] -= E @ U[i1:i2, i2:]

    packed = pack_nibbles_device(Q.t())
    return QuantizedWeight(packed.cpu(), scales.to(torch.float16).cpu().contiguous(), G, K, N)


def find_decoder_blocks(model: nn.Module) -> Optional[nn.ModuleList]:
    """The repeated transformer blocks of a causal LM, looked up under the
    attribute paths of the common model families (reference gptq.py:178-189):
    Llama / Mistral (``model.layers``), GPT-2 (``transformer.h``), OPT
    (``model.decoder.layers``), GPT-NeoX (``gpt_neox.layers``)."""
    for path in ("model.layers", "transformer.h", "model.decoder.layers", "gpt_neox.layers"):
        node = model
        for attr in path.split("."):
            node = getattr(node, attr, None)
            if node is None:
                break
        if isinstance(node, (nn.ModuleList, list)) and len(node) > 0:
            return node
    return None


def supported_linear(lin: nn.Linear, group_size: int) -> bool:
    """Whether the kernels take this layer's shape (reference gptq.py:192-194)."""
    K, N = lin.in_features, lin.out_features
    return K % group_size == 0 and N % 4 == 0 and K % 32 == 0


def _hessian_hook(acc: HessianAccumulator):
    def hook(_module, args):
        if args and isinstance(args[0], torch.Tensor):
            acc.add(args[0].detach())
        return None
    return hook


def _replace(root: nn.Module, dotted: str, module: nn.Module) -> None:
    *parents, leaf = dotted.split(".")
    for name in parents:
        root = getattr(root, name)
    setattr(root, leaf, module)


@torch.no_grad()
def quantize_model_gptq(model: nn.Module, calibration: Iterable[torch.Tensor],
                        group_size: int = 128, damp: float = 0.01,
                        make_quant_linear: Optional[Callable] = None,
                        log: Callable[[str], None] = print) -> Tuple[int, List[str]]:
    """Quantises a causal LM in place, one decoder block at a time (reference
    gptq.py:197-261).

    For each block: forward pre-hooks accumulate every supported linear's
    input Hessian over the calibration batches, then each such linear is
    replaced by a :class:`~nibblegemm_amd.ops.QuantLinear` of its GPTQ weights.
    A block is calibrated after the blocks before it were replaced, so it sees
    the activations the quantised model produces.  Returns ``(replaced,
    skipped)``, the latter naming the linears whose shapes the kernels do not
    take."""
    make = make_quant_linear or (lambda qw, bias: QuantLinear(qw, bias))
    blocks = find_decoder_blocks(model)
    if blocks is None:
        raise RuntimeError("could not locate decoder blocks on this model")
    batches = list(calibration)
    device = next(model.parameters()).device
    replaced, skipped = 0, []
    for b, block in enumerate(blocks):
        targets: Dict[str, nn.Linear] = {}
        for name, mod in block.named_modules():
            if isinstance(mod, nn.Linear):
                if supported_linear(mod, group_size):
                    targets[name] = mod
                else:
                    skipped.append(f"block{b}.{name} [{mod.in_features}x{mod.out_features}]")
        if not targets:
            continue
        accs = {name: HessianAccumulator(lin.in_features, device) for name, lin in targets.items()}
        hooks = [lin.register_forward_pre_hook(_hessian_hook(accs[name]))
                 for name, lin in targets.items()]
        try:
            for batch in batches:
                model(batch.to(device))
        finally:
            for h in hooks:
                h.remove()
        for name, lin in targets.items():
            qw = gptq_quantize(lin.weight.data.t().contiguous(), accs[name].H,
                               group_size=group_size, damp=damp)
            bias = lin.bias.data.clone() if lin.bias is not None else None
            _replace(block, name, make(qw.to(device), bias))
            replaced += 1
        del accs
        log(f"  block {b + 1}/{len(blocks)}: {len(targets)} layers quantised")
    return replaced, skipped
