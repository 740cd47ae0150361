"""Cut Cross-Entropy (fused lm_head projection + cross-entropy) on MI355X.

Drop-in for ``chronicals.kernels.cut_cross_entropy`` (reference
chronicals/kernels/cut_cross_entropy.py): same public names, argument order,
defaults and loss semantics, with the compute in hand-written gfx950 HIP
kernels (``libchronicals_cce.so``, C ABI in include/chronicals_cce.h).

Differences from the reference, all deliberate:
  * ``reduction`` keyword ('mean' | 'sum' | 'none'), with the semantics of the
    reference's sibling ``fused_linear_cross_entropy``
    (triton_kernels.py:2481-2491).  ``CutCrossEntropyLoss`` accepts all three
    (the reference raises for anything but 'mean', cut_cross_entropy.py:1120).
  * The backward applies the one-hot term of dLoss/dlogits, which the
    reference's CPU backward loses (cut_cross_entropy.py:773-780); its GPU path
    (:530-546) applies it.
  * Tensors must live on a HIP device; there is no CPU path.  hidden and weight
    are computed in bf16 with fp32 accumulation (fp16/fp32 inputs are rounded
    to bf16 at the boundary); gradients come back in the input dtypes (:808).
  * ``use_triton`` is accepted and ignored: there is one HIP path.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from .. import _lib
from .. import ops as _ops  # noqa: F401  (registers chronicals_hip::cce_fwd / cce_bwd)
from .logits_cross_entropy import ChunkedCrossEntropyLoss, chunked_cross_entropy_loss  # noqa: F401

# Constants of the reference module (cut_cross_entropy.py:45-56), kept for
# import compatibility.  The chunk size is the vocabulary band width of the
# backward pass here.
CHUNK_SIZE_SMALL_VOCAB = 4096
CHUNK_SIZE_MEDIUM_VOCAB = 8192
CHUNK_SIZE_LARGE_VOCAB = 16384
DEFAULT_VOCAB_CHUNK_SIZE = 8192
TRITON_BLOCK_SIZE = 4096
TRITON_BLOCK_SIZE_MAX = 65536 // 2

__all__ = [
    "cut_cross_entropy",
    "linear_cross_entropy",
    "cce_forward_pytorch",
    "cce_backward_pytorch",
    "chunked_cross_entropy_loss",
    "ChunkedCrossEntropyLoss",
    "CutCrossEntropyLoss",
    "CutCrossEntropyFunction",
    "CutCrossEntropyForward",
    "CutCrossEntropyBackward",
    "AdaptiveCrossEntropyLoss",
    "get_optimal_chunk_size",
    "estimate_memory_savings",
    "compute_z_loss",
]


def get_optimal_chunk_size(vocab_size: int, hidden_dim: int, available_vram_gb: float = 40.0) -> int:
    """Power-of-two vocabulary chunk for a vocabulary size.

    Same rule as the reference (cut_cross_entropy.py:59-90): 4096 below 64K
    entries, 8192 below 128K, 16384 above, capped by 80% of
    ``available_vram_gb`` over 8*hidden_dim bytes per entry, at least 256.
    """
    usable = available_vram_gb * 0.8 * 1024 ** 3
    max_chunk = int(usable / (8 * hidden_dim))
    if vocab_size < 64000:
        optimal = min(max_chunk, CHUNK_SIZE_SMALL_VOCAB)
    elif vocab_size < 128000:
        optimal = min(max_chunk, CHUNK_SIZE_MEDIUM_VOCAB)
    else:
        optimal = min(max_chunk, CHUNK_SIZE_LARGE_VOCAB)
    return max(256, 2 ** int(math.log2(optimal)))


def _as_bf16_rows(x: torch.Tensor) -> torch.Tensor:
    """Contiguous bf16 copy/view of a 2-D tensor (the op itself realigns a
    storage offset that is not 16-byte aligned)."""
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    return x.contiguous()


def _validate(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, bias: Optional[torch.Tensor]):
    if not (hidden.is_cuda and weight.is_cuda and labels.is_cuda):
        raise RuntimeError(
            "chronicals_amd cut_cross_entropy runs only on HIP devices: hidden, weight and labels must be "
            f"device tensors (got {hidden.device}, {weight.device}, {labels.device})"
        )
    if hidden.device != weight.device or hidden.device != labels.device:
        raise RuntimeError("hidden, weight and labels must be on the same device")
    if weight.dim() != 2:
        raise RuntimeError(f"weight must be [vocab_size, hidden_dim], got shape {tuple(weight.shape)}")
    if hidden.dim() < 1 or hidden.shape[-1] != weight.shape[1]:
        raise RuntimeError(
            f"hidden last dim {tuple(hidden.shape)[-1:]} does not match weight hidden_dim {weight.shape[1]}"
        )
    if labels.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"labels must be int64 or int32, got {labels.dtype}")
    n = hidden.numel() // hidden.shape[-1] if hidden.shape[-1] else 0
    if labels.numel() != n:
        raise RuntimeError(f"labels has {labels.numel()} elements but hidden has {n} rows")
    if bias is not None:
        if bias.dim() != 1 or bias.shape[0] != weight.shape[0]:
            raise RuntimeError(f"bias must be [vocab_size={weight.shape[0]}], got {tuple(bias.shape)}")
        if bias.device != hidden.device:
            raise RuntimeError("bias must be on the same device as hidden")
    if hidden.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise RuntimeError(f"hidden dtype {hidden.dtype} not supported (bf16, fp16, fp32)")
    if weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise RuntimeError(f"weight dtype {weight.dtype} not supported (bf16, fp16, fp32)")


def _reduction_code(reduction: str) -> int:
    try:
        return _lib.REDUCTIONS[reduction]
    except KeyError:
        raise ValueError(f"reduction must be 'mean', 'sum' or 'none', got {reduction!r}") from None


def _forward_raw(hidden, weight, labels, bias, ignore_index, label_smoothing, z_loss_weight, red,
                 smoothing_form=_lib.CCE_SMOOTH_LOGV, lse_rows=_lib.CCE_LSE_ALL_ROWS):
    """Operand preparation + one chronicals_hip::cce_fwd call.

    Returns (loss, lse, n_valid, h2, w2, lab, b32, target): the bf16 [N, d] /
    [V, d] operands, flat labels and fp32 bias the backward reuses, and the
    per-row target logits.  With lse_rows = CCE_LSE_LABELLED_ROWS the ignored
    rows' lse and target are 0 and the forward skips their share of the
    logits GEMM; callers that only use labelled rows' lse pass it.
    """
    _validate(hidden, weight, labels, bias)
    d = hidden.shape[-1]
    h2 = _as_bf16_rows(hidden.detach().reshape(-1, d))
    w2 = _as_bf16_rows(weight.detach())
    lab = labels.reshape(-1)
    if not lab.is_contiguous():
        lab = lab.contiguous()
    b32 = None if bias is None else bias.detach().to(torch.float32).contiguous()
    loss, lse, n_valid, target = torch.ops.chronicals_hip.cce_fwd(h2, w2, lab, b32, int(ignore_index),
                                                                  float(label_smoothing), float(z_loss_weight),
                                                                  int(smoothing_form), int(red), int(lse_rows))
    return loss, lse, n_valid, h2, w2, lab, b32, target


class CutCrossEntropyFunction(torch.autograd.Function):
    """Autograd contract of the reference (cut_cross_entropy.py:815-858).

    forward(hidden, weight, labels, bias, chunk_size, ignore_index,
            label_smoothing, z_loss_weight, reduction) -> loss
    Saves only the bf16 operands, labels, lse [N] and n_valid (O(N) extra).
    """

    @staticmethod
    def forward(ctx, hidden, weight, labels, bias, chunk_size, ignore_index, label_smoothing, z_loss_weight,
                reduction="mean"):
        red = _reduction_code(reduction)
        loss, lse, n_valid, h2, w2, lab, b32, _ = _forward_raw(hidden, weight, labels, bias, ignore_index,
                                                               label_smoothing, z_loss_weight, red,
                                                               lse_rows=_lib.CCE_LSE_LABELLED_ROWS)
        ctx.save_for_backward(h2, w2, lab, lse, n_valid, b32)
        ctx.cfg = (int(chunk_size), int(ignore_index), float(label_smoothing), float(z_loss_weight), red)
        ctx.shapes = (hidden.shape, hidden.dtype, weight.dtype, None if bias is None else bias.dtype)
        if red == _lib.CCE_REDUCTION_NONE:
            return loss.view(labels.shape)
        return loss.view(())

    @staticmethod
    def backward(ctx, grad_output):
        dh, dw, db = _backward_raw(ctx, grad_output, ctx.needs_input_grad[0], ctx.needs_input_grad[1],
                                   ctx.needs_input_grad[3])
        return dh, dw, None, db, None, None, None, None, None


def _backward_raw(ctx, grad_output, need_dh, need_dw, need_db):
    """One chronicals_hip::cce_bwd call from what _forward_raw's caller saved
    (ctx.saved_tensors = (h2, w2, lab, lse, n_valid, b32), ctx.cfg, ctx.shapes);
    returns (dH, dW, dB) in the input dtypes, None where not requested."""
    h2, w2, lab, lse, n_valid, b32 = ctx.saved_tensors
    chunk_size, ignore_index, eps, zw, red = ctx.cfg
    hshape, hdtype, wdtype, bdtype = ctx.shapes
    need_db = b32 is not None and need_db
    if not (need_dh or need_dw or need_db):
        return None, None, None
    # bf16 inputs get bf16 gradients; fp16 / fp32 inputs get them from fp32
    dh, dw, db = torch.ops.chronicals_hip.cce_bwd(
        grad_output, h2, w2, lab, lse, n_valid, b32, ignore_index, eps, zw, red, chunk_size,
        need_dh, need_dw, need_db, hdtype != torch.bfloat16, wdtype != torch.bfloat16)
    dh = dh.view(hshape).to(hdtype) if need_dh else None
    dw = dw.to(wdtype) if need_dw else None
    db = db.to(bdtype) if need_db else None
    return dh, dw, db


class _LinearCE(torch.autograd.Function):
    """(loss, lse) of the fused kernels; lse carries no gradient and is 0 on
    ignored rows (the forward skips them).

    apply(hidden, weight, labels, bias, chunk_size, ignore_index, eps, z,
          reduction_code, smoothing_form)
    """

    @staticmethod
    def forward(ctx, hidden, weight, labels, bias, chunk_size, ignore_index, eps, z, red, form):
        loss, lse, n_valid, h2, w2, lab, b32, _ = _forward_raw(hidden, weight, labels, bias, ignore_index, eps, z, red,
                                                            form, _lib.CCE_LSE_LABELLED_ROWS)
        ctx.save_for_backward(h2, w2, lab, lse, n_valid, b32)
        ctx.cfg = (int(chunk_size), int(ignore_index), float(eps), float(z), red)
        ctx.shapes = (hidden.shape, hidden.dtype, weight.dtype, None if bias is None else bias.dtype)
        ctx.mark_non_differentiable(lse)
        out = loss.view(labels.shape) if red == _lib.CCE_REDUCTION_NONE else loss.view(())
        return out, lse

    @staticmethod
    def backward(ctx, grad_loss, grad_lse):
        del grad_lse
        dh, dw, db = _backward_raw(ctx, grad_loss, ctx.needs_input_grad[0], ctx.needs_input_grad[1],
                                   ctx.needs_input_grad[3])
        return dh, dw, None, db, None, None, None, None, None, None


class CutCrossEntropyForward:
    """The reference's forward pass as a static method (cut_cross_entropy.py:559-692), on cce_forward."""

    @staticmethod
    def forward(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, bias: Optional[torch.Tensor] = None,
                chunk_size: int = 8192, ignore_index: int = -100, label_smoothing: float = 0.0,
                z_loss_weight: float = 0.0, use_kahan: bool = True):
        """(loss, logsumexp [N], target_logit [N], valid_mask [N]); 'mean' loss, no autograd.
        ``use_kahan`` is accepted: the kernels merge fp32 partials in a fixed order."""
        del chunk_size, use_kahan
        with torch.no_grad():
            loss, lse, _, _, _, lab, _, target = _forward_raw(hidden, weight, labels, bias, ignore_index,
                                                              label_smoothing, z_loss_weight,
                                                              _lib.CCE_REDUCTION_MEAN)
        return loss.view(()), lse, target, lab != ignore_index


class CutCrossEntropyBackward:
    """The reference's backward pass as a static method (cut_cross_entropy.py:695-808), on cce_backward."""

    @staticmethod
    def backward(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, logsumexp: torch.Tensor,
                 valid_mask: torch.Tensor, grad_output: torch.Tensor, bias: Optional[torch.Tensor] = None,
                 chunk_size: int = 8192, ignore_index: int = -100, label_smoothing: float = 0.0,
                 z_loss_weight: float = 0.0):
        """(grad_hidden, grad_weight, grad_bias or None) of the 'mean' loss times grad_output.

        Rows where ``valid_mask`` is False are treated as ignored.  A scalar
        grad_output scales every row by grad_output / n_valid; a per-row one
        scales row n by grad_output[n] / n_valid (:745).  The one-hot term is
        applied (the reference's CPU path loses it at :773-780).
        """
        _validate(hidden, weight, labels, bias)
        d = hidden.shape[-1]
        with torch.no_grad():
            h2 = _as_bf16_rows(hidden.detach().reshape(-1, d))
            w2 = _as_bf16_rows(weight.detach())
            vm = valid_mask.reshape(-1).to(torch.bool)
            lab = torch.where(vm, labels.reshape(-1).to(torch.int64),
                              torch.full_like(vm, int(ignore_index), dtype=torch.int64)).contiguous()
            n_valid = vm.sum().to(torch.int32).reshape(1)
            b32 = None if bias is None else bias.detach().to(torch.float32).contiguous()
            lse = logsumexp.detach().reshape(-1).to(torch.float32).contiguous()
            g = torch.as_tensor(grad_output, device=h2.device).detach().to(torch.float32)
            if g.numel() == 1:
                red = _lib.CCE_REDUCTION_MEAN
            else:
                red = _lib.CCE_REDUCTION_NONE
                g = g.reshape(-1) / n_valid.clamp(min=1).to(torch.float32)
            dh, dw, db = torch.ops.chronicals_hip.cce_bwd(
                g, h2, w2, lab, lse, n_valid, b32, int(ignore_index), float(label_smoothing), float(z_loss_weight),
                red, int(chunk_size), True, True, b32 is not None, hidden.dtype != torch.bfloat16,
                weight.dtype != torch.bfloat16)
        return (dh.view(hidden.shape).to(hidden.dtype), dw.to(weight.dtype),
                db.to(bias.dtype) if bias is not None else None)


def cut_cross_entropy(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    labels: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    chunk_size: int = 8192,
    ignore_index: int = -100,
    label_smoothing: float = 0.0,
    z_loss_weight: float = 0.0,
    use_triton: bool = True,
    reduction: str = "mean",
) -> torch.Tensor:
    """Fused lm_head projection + cross-entropy without materialising logits.

    Signature and defaults of the reference (cut_cross_entropy.py:1023-1033)
    plus ``reduction``.  hidden [B,S,d] or [N,d]; weight [V,d]; labels [B,S]
    or [N] (int64/int32); bias [V] or None.  Returns a 0-dim fp32 loss for
    'mean'/'sum' and a labels-shaped fp32 tensor for 'none'.  The loss of a
    row is (1-eps)*(lse - target) + eps*log(V) + z*lse^2 (reference
    :671-683); rows labelled ``ignore_index`` contribute 0 and are excluded
    from the mean's denominator max(n_valid, 1) (:686-690).
    """
    del use_triton  # single HIP path
    return CutCrossEntropyFunction.apply(hidden, weight, labels, bias, chunk_size, ignore_index, label_smoothing,
                                         z_loss_weight, reduction)


def linear_cross_entropy(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    labels: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    ignore_index: int = -100,
    reduction: str = "mean",
    *,
    chunk_size: int = DEFAULT_VOCAB_CHUNK_SIZE,
    label_smoothing: float = 0.0,
    z_loss_weight: float = 0.0,
) -> torch.Tensor:
    """``cut_cross_entropy`` in the (hidden, weight, labels, bias, ignore_index,
    reduction) argument order.

    The reference imports this name from its cut_cross_entropy module
    (chronicals_trainer.py:79-89, triton_kernels.py:44-58) but never defines
    it, so those imports fail there and the trainer falls back to its
    non-fused losses.  Here the name exists, so the same import block
    resolves against this package.
    """
    return CutCrossEntropyFunction.apply(hidden, weight, labels, bias, chunk_size, ignore_index, label_smoothing,
                                         z_loss_weight, reduction)


# The static forward / backward passes under the names triton_kernels.py:50-51
# imports from the reference module (which does not define them either).
cce_forward_pytorch = CutCrossEntropyForward.forward
cce_backward_pytorch = CutCrossEntropyBackward.backward


class CutCrossEntropyLoss(nn.Module):
    """nn.Module wrapper (reference cut_cross_entropy.py:1081-1162).

    ``chunk_size=None`` picks ``get_optimal_chunk_size(V, d)`` per call, as
    the reference does (:1143-1146).  Accepts reduction 'mean', 'sum' or
    'none'.
    """

    def __init__(self, chunk_size: Optional[int] = None, ignore_index: int = -100, label_smoothing: float = 0.0,
                 z_loss_weight: float = 0.0, reduction: str = "mean"):
        super().__init__()
        _reduction_code(reduction)
        self.chunk_size = chunk_size
        self.ignore_index = ignore_index
        self.label_smoothing = label_smoothing
        self.z_loss_weight = z_loss_weight
        self.reduction = reduction

    def forward(self, hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.chunk_size is None:
            chunk_size = get_optimal_chunk_size(weight.shape[0], weight.shape[1])
        else:
            chunk_size = self.chunk_size
        return cut_cross_entropy(hidden, weight, labels, bias, chunk_size, self.ignore_index, self.label_smoothing,
                                 self.z_loss_weight, reduction=self.reduction)

    def extra_repr(self) -> str:
        return (f"chunk_size={self.chunk_size}, ignore_index={self.ignore_index}, "
                f"label_smoothing={self.label_smoothing}, z_loss_weight={self.z_loss_weight}")


class AdaptiveCrossEntropyLoss(nn.Module):
    """Picks the cross-entropy form by vocabulary size (reference cut_cross_entropy.py:1283-1372).

    forward(hidden, weight, labels, bias=None) or forward(logits, labels).
    Below ``small_vocab_threshold`` the reference uses torch's
    nn.CrossEntropyLoss (uniform-target label smoothing, no z-loss, mean over
    the non-ignored rows); at or above it, CutCrossEntropyLoss (hidden) or
    chunked_cross_entropy_loss (logits).  Every branch runs on the HIP
    kernels: the small-vocabulary ones with the uniform smoothing form and
    z = 0.  With every label ignored the small-vocabulary branches return 0
    (torch's mean is NaN there).
    """

    def __init__(self, small_vocab_threshold: int = 32000, large_vocab_threshold: int = 100000,
                 ignore_index: int = -100, label_smoothing: float = 0.0, z_loss_weight: float = 0.0):
        super().__init__()
        self.small_vocab_threshold = small_vocab_threshold
        self.large_vocab_threshold = large_vocab_threshold
        self.ignore_index = ignore_index
        self.label_smoothing = label_smoothing
        self.z_loss_weight = z_loss_weight
        self.cce = CutCrossEntropyLoss(ignore_index=ignore_index, label_smoothing=label_smoothing,
                                       z_loss_weight=z_loss_weight)

    def forward(self, hidden_or_logits: torch.Tensor, weight_or_labels: torch.Tensor,
                labels_or_none: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        from .logits_cross_entropy import LogitsCrossEntropyFunction, _rows
        if labels_or_none is not None:
            hidden, weight, labels = hidden_or_logits, weight_or_labels, labels_or_none
            if weight.shape[0] < self.small_vocab_threshold:
                loss, _ = _LinearCE.apply(hidden, weight, labels, bias, 8192, self.ignore_index,
                                          self.label_smoothing, 0.0, _lib.CCE_REDUCTION_MEAN,
                                          _lib.CCE_SMOOTH_UNIFORM)
                return loss
            return self.cce(hidden, weight, labels, bias)
        logits, labels = hidden_or_logits, weight_or_labels
        if logits.shape[-1] < self.small_vocab_threshold:
            x, lab = _rows(logits, labels, "AdaptiveCrossEntropyLoss")
            return LogitsCrossEntropyFunction.apply(x, lab, self.ignore_index, self.label_smoothing, 0.0,
                                                    _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_REDUCTION_MEAN)
        return chunked_cross_entropy_loss(logits, labels, ignore_index=self.ignore_index,
                                          label_smoothing=self.label_smoothing, z_loss_weight=self.z_loss_weight)


def compute_z_loss(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                   bias: Optional[torch.Tensor] = None, ignore_index: int = -100,
                   chunk_size: int = 8192) -> torch.Tensor:
    """Mean over valid rows of lse^2 (reference cut_cross_entropy.py:1379-1400).

    A monitoring value: it is returned without autograd history.  The
    reference computes it with its plain-torch forward, which autograd would
    track on its CPU path; the fused kernels here have no gradient for the
    z-loss term alone.  ``chunk_size`` is accepted for signature
    compatibility.
    """
    del chunk_size
    _, lse, _, _, _, lab, _, _ = _forward_raw(hidden, weight, labels, bias, ignore_index, 0.0, 0.0,
                                              _lib.CCE_REDUCTION_MEAN, lse_rows=_lib.CCE_LSE_LABELLED_ROWS)
    valid = (lab != ignore_index).to(torch.float32)
    return (lse * lse * valid).sum() / valid.sum().clamp(min=1)


def estimate_memory_savings(batch_size: int, seq_len: int, vocab_size: int, chunk_size: int = 8192) -> dict:
    """Analytic MB estimate of the reference (cut_cross_entropy.py:1403-1430).

    Standard = N*V*4*2 bytes (fp32 logits and their gradient); chunked =
    N*chunk*4*2 bytes.
    """
    batch_seq = batch_size * seq_len
    standard_mb = batch_seq * vocab_size * 4 * 2 / (1024 ** 2)
    cce_mb = batch_seq * chunk_size * 4 * 2 / (1024 ** 2)
    return {
        "standard_mb": standard_mb,
        "cce_mb": cce_mb,
        "reduction_factor": standard_mb / cce_mb,
        "savings_mb": standard_mb - cce_mb,
    }
