"""Cross-entropy over logits that already exist, on MI355X.

The callers that hold a [N, V] logits tensor (a model that returns logits,
evaluation) use one of three reference entry points, all served here by HIP
row kernels (``cce_logits_forward`` / ``cce_logits_backward`` /
``cce_logits_forward_backward`` in include/chronicals_cce.h).  The forward
reads the logits once (online max / sum-exp, target gather, row sum); the
autograd backward reads them again and writes the gradient with grad_output
folded in.  Where the reference computes the gradient inside its forward
(``liger_cross_entropy_forward(compute_grads=True)``, ``fused_cross_entropy``)
one kernel does both, re-reading each row from the memory-side cache.

  chunked_cross_entropy_loss, ChunkedCrossEntropyLoss
      reference chronicals/kernels/cut_cross_entropy.py:1169-1277.  Label
      smoothing in the reference's form (1-eps)*ce + eps*log(V)
      (CCE_SMOOTH_LOGV); the gradient is what autograd gives through that
      expression.
  liger_cross_entropy, liger_cross_entropy_forward, liger_cross_entropy_backward,
  LigerCrossEntropyFunction
      reference chronicals/kernels/triton_kernels.py:2839-3125.  Uniform-target
      label smoothing (1-eps)*ce + eps*(lse - mean(x)) (CCE_SMOOTH_UNIFORM).
  fused_cross_entropy, fused_cross_entropy_triton
      reference triton_kernels.py:141-257 and :2206-2218.  Returns the mean
      loss and the per-row (unnormalised) gradient in fp32, as the reference
      kernel does.
  compute_padding_free_loss, compute_packed_loss
      reference chronicals/data/sequence_packer.py:1660-1717 and
      sequence_packer_v2.py:1058-1113: the packed-sequence losses, torch's
      label-smoothed cross-entropy (the uniform form) per token, weighted by an
      optional ``loss_mask`` and divided by its sum ('mean').

Deliberate differences from the reference:
  * Tensors must live on a HIP device; there is no CPU path.
  * ``chunked_cross_entropy_loss`` also accepts [N, V] logits and a
    ``reduction`` keyword ('mean' default, 'sum', 'none'); ``chunk_size`` is
    accepted and unused (each row is streamed whole).
  * A label outside [0, V) that is not ``ignore_index`` contributes lse with
    no target term (the chunked reference's gather raises instead).
  * ``LigerCrossEntropyFunction`` computes the gradient in backward, with the
    incoming gradient folded in, instead of cloning the logits in forward and
    rescaling them in backward: same values, one [N, V] buffer fewer.
  * With every label ignored, ``liger_cross_entropy_forward`` returns a zero
    gradient (the reference returns the logits unchanged, :3026-3027, which is
    no gradient of the zero loss).
  * Losses are fp32 whatever the logits' dtype (torch's cross_entropy, which
    the packed-sequence losses call, returns the logits' dtype).
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn

from .. import _lib
from .. import ops as _ops  # noqa: F401  (registers chronicals_hip::ce_logits_*)

__all__ = [
    "chunked_cross_entropy_loss",
    "ChunkedCrossEntropyLoss",
    "liger_cross_entropy",
    "liger_cross_entropy_forward",
    "liger_cross_entropy_backward",
    "LigerCrossEntropyFunction",
    "fused_cross_entropy",
    "fused_cross_entropy_triton",
    "LogitsCrossEntropyFunction",
    "compute_padding_free_loss",
    "compute_packed_loss",
]

TRITON_BLOCK_SIZE_MAX = 65536 // 2  # reference triton_kernels.py:2835, kept for import compatibility


def _reduction_code(reduction: str) -> int:
    try:
        return _lib.REDUCTIONS[reduction]
    except KeyError:
        raise ValueError(f"reduction must be 'mean', 'sum' or 'none', got {reduction!r}") from None


def _rows(logits: torch.Tensor, labels: torch.Tensor, what: str) -> Tuple[torch.Tensor, torch.Tensor]:
    """[..., V] logits and [...] labels as [N, V] (last dimension contiguous) and [N]."""
    if not (logits.is_cuda and labels.is_cuda):
        raise RuntimeError(f"chronicals_amd {what} runs only on HIP devices: logits and labels must be device "
                           f"tensors (got {logits.device}, {labels.device})")
    if logits.dim() < 2:
        raise RuntimeError(f"logits must be [..., V], got shape {tuple(logits.shape)}")
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    # the kernels take unit-stride rows that do not overlap (row stride >= V)
    if (V > 1 and x.stride(-1) != 1) or (x.shape[0] > 1 and x.stride(0) < V):
        x = x.contiguous()
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        x = x.float()
    lab = labels.reshape(-1)
    if lab.numel() != x.shape[0]:
        raise RuntimeError(f"labels has {lab.numel()} elements but logits has {x.shape[0]} rows")
    if lab.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"labels must be int64 or int32, got {lab.dtype}")
    return x, lab.contiguous()


class LogitsCrossEntropyFunction(torch.autograd.Function):
    """Autograd over chronicals_hip::ce_logits_fwd / ce_logits_bwd.

    apply(logits2d, labels, ignore_index, label_smoothing, z_loss_weight,
          smoothing_form, reduction_code) -> loss (scalar, or [N] for 'none').
    The forward keeps only lse [N] and n_valid beyond the inputs; the
    backward streams the logits once more and writes dLoss/dlogits scaled by
    the incoming gradient.
    """

    @staticmethod
    def forward(ctx, logits2d, labels, ignore_index, label_smoothing, z_loss_weight, smoothing_form, red):
        loss, lse, n_valid = torch.ops.chronicals_hip.ce_logits_fwd(
            logits2d, labels, int(ignore_index), float(label_smoothing), float(z_loss_weight), int(smoothing_form),
            int(red))
        ctx.save_for_backward(logits2d, labels, lse, n_valid)
        ctx.cfg = (int(ignore_index), float(label_smoothing), float(z_loss_weight), int(smoothing_form), int(red))
        return loss if red == _lib.CCE_REDUCTION_NONE else loss.view(())

    @staticmethod
    def backward(ctx, grad_output):
        if not ctx.needs_input_grad[0]:
            return (None,) * 7
        logits2d, labels, lse, n_valid = ctx.saved_tensors
        ignore_index, eps, zw, form, red = ctx.cfg
        dx = torch.ops.chronicals_hip.ce_logits_bwd(grad_output, logits2d, labels, lse, n_valid, ignore_index, eps,
                                                    zw, form, red, False)
        return dx, None, None, None, None, None, None


# ---------------------------------------------------------------------------
# cut_cross_entropy.py:1169-1277
# ---------------------------------------------------------------------------

def chunked_cross_entropy_loss(
    logits: torch.Tensor,
    labels: torch.Tensor,
    chunk_size: int = 8192,
    ignore_index: int = -100,
    label_smoothing: float = 0.0,
    z_loss_weight: float = 0.0,
    reduction: str = "mean",
) -> torch.Tensor:
    """Cross-entropy over pre-computed logits (reference cut_cross_entropy.py:1169-1249).

    logits [batch, seq, V] (or [N, V]), labels [batch, seq] (or [N]).  Per
    row whose label is not ``ignore_index``:
    (1-eps)*(lse - logit[label]) + eps*log(V) + z*lse^2, with
    lse = log(sum exp(logits) + 1e-10); 'mean' divides the sum by
    max(n_valid, 1).  Differentiable in ``logits``.
    """
    del chunk_size
    red = _reduction_code(reduction)
    x, lab = _rows(logits, labels, "chunked_cross_entropy_loss")
    loss = LogitsCrossEntropyFunction.apply(x, lab, ignore_index, label_smoothing, z_loss_weight,
                                            _lib.CCE_SMOOTH_LOGV, red)
    return loss.view(labels.shape) if red == _lib.CCE_REDUCTION_NONE else loss


class ChunkedCrossEntropyLoss(nn.Module):
    """Module form of chunked_cross_entropy_loss (reference cut_cross_entropy.py:1252-1277)."""

    def __init__(self, chunk_size: int = 8192, ignore_index: int = -100, label_smoothing: float = 0.0,
                 z_loss_weight: float = 0.0):
        super().__init__()
        self.chunk_size = chunk_size
        self.ignore_index = ignore_index
        self.label_smoothing = label_smoothing
        self.z_loss_weight = z_loss_weight

    def forward(self, logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
        return chunked_cross_entropy_loss(logits, labels, self.chunk_size, self.ignore_index,
                                          self.label_smoothing, self.z_loss_weight)


# ---------------------------------------------------------------------------
# triton_kernels.py:2839-3125 (Liger-style row kernel)
# ---------------------------------------------------------------------------

def liger_cross_entropy_forward(
    logits: torch.Tensor,
    target: torch.Tensor,
    ignore_index: int = -100,
    lse_square_scale: float = 0.0,
    label_smoothing: float = 0.0,
    reduction: str = "mean",
    compute_grads: bool = True,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Loss and (optionally) the gradient written over the logits.

    Reference triton_kernels.py:2979-3067.  Per valid row
    (1-eps)*(lse - x[target]) + eps*(lse - mean(x)) + s*lse^2, divided by
    n_valid for 'mean'; 'none' returns the per-row losses, otherwise their
    sum.  With ``compute_grads`` the logits ([N, V], or the contiguous copy
    made when the last dimension is strided) are overwritten with
    dLoss/dlogits (divided by n_valid for 'mean'), and returned.
    """
    red = _reduction_code(reduction)
    x, lab = _rows(logits, target, "liger_cross_entropy_forward")
    if compute_grads:
        # one kernel: loss and gradient, written over the logits; only 'mean'
        # gradients are divided by n_valid (triton_kernels.py:2946-2947)
        loss, _, _ = torch.ops.chronicals_hip.ce_logits_fwd_bwd_(
            x, lab, int(ignore_index), float(label_smoothing), float(lse_square_scale), _lib.CCE_SMOOTH_UNIFORM, red,
            red == _lib.CCE_REDUCTION_MEAN)
    else:
        loss, _, _ = torch.ops.chronicals_hip.ce_logits_fwd(
            x, lab, int(ignore_index), float(label_smoothing), float(lse_square_scale), _lib.CCE_SMOOTH_UNIFORM, red)
    return (loss if red == _lib.CCE_REDUCTION_NONE else loss.view(())), x


def liger_cross_entropy_backward(logits: torch.Tensor, grad_out: torch.Tensor) -> torch.Tensor:
    """Scale gradients left in ``logits`` by liger_cross_entropy_forward (reference :3070-3086)."""
    if grad_out.numel() == 1:
        return logits.mul_(grad_out.reshape(()).to(logits.dtype))
    return logits.mul_(grad_out.reshape(-1, 1).to(logits.dtype))


class LigerCrossEntropyFunction(torch.autograd.Function):
    """Autograd for the uniform-smoothing row kernels (reference triton_kernels.py:3089-3106).

    apply(logits, target, ignore_index=-100, lse_scale=0.0, label_smoothing=0.0,
    reduction='mean').  The reference computes the gradient in forward into a
    clone of the logits and rescales it in backward; here the backward writes
    it once, with grad_output folded in.
    """

    @staticmethod
    def forward(ctx, logits, target, ignore_index=-100, lse_scale=0.0, label_smoothing=0.0, reduction="mean"):
        red = _reduction_code(reduction)
        x, lab = _rows(logits, target, "liger_cross_entropy")
        loss, lse, n_valid = torch.ops.chronicals_hip.ce_logits_fwd(
            x, lab, int(ignore_index), float(label_smoothing), float(lse_scale), _lib.CCE_SMOOTH_UNIFORM, red)
        ctx.save_for_backward(x, lab, lse, n_valid)
        ctx.cfg = (int(ignore_index), float(label_smoothing), float(lse_scale), red)
        ctx.shape = logits.shape
        return loss if red == _lib.CCE_REDUCTION_NONE else loss.view(())

    @staticmethod
    def backward(ctx, grad_output):
        if not ctx.needs_input_grad[0]:
            return (None,) * 6
        x, lab, lse, n_valid = ctx.saved_tensors
        ignore_index, eps, zw, red = ctx.cfg
        dx = torch.ops.chronicals_hip.ce_logits_bwd(grad_output, x, lab, lse, n_valid, ignore_index, eps, zw,
                                                    _lib.CCE_SMOOTH_UNIFORM, red, False)
        return dx.view(ctx.shape), None, None, None, None, None


def liger_cross_entropy(
    logits: torch.Tensor,
    target: torch.Tensor,
    ignore_index: int = -100,
    lse_square_scale: float = 0.0,
    label_smoothing: float = 0.0,
    reduction: str = "mean",
) -> torch.Tensor:
    """Differentiable uniform-smoothing cross-entropy (reference triton_kernels.py:3109-3125)."""
    return LigerCrossEntropyFunction.apply(logits, target, ignore_index, lse_square_scale, label_smoothing,
                                           reduction)


# ---------------------------------------------------------------------------
# triton_kernels.py:141-257, :2206-2218
# ---------------------------------------------------------------------------

def fused_cross_entropy_triton(
    logits: torch.Tensor,
    labels: torch.Tensor,
    label_smoothing: float = 0.0,
    z_loss_weight: float = 1e-4,
    ignore_index: int = -100,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Mean loss and fp32 per-row gradient (reference triton_kernels.py:213-257).

    logits [batch, seq, V].  Loss: the sum over valid rows of
    (1-eps)*(lse - x[label]) + eps*(lse - mean(x)) + z*lse^2, divided by
    max(n_valid, 1).  dlogits (fp32, shape of logits): each valid row's
    p*(1 + 2z*lse) - eps/V - (1-eps)*onehot, not divided by n_valid (as the
    reference kernel stores it); zero rows for ignored labels.
    """
    x, lab = _rows(logits, labels, "fused_cross_entropy")
    # one kernel, as the reference's: mean loss, unscaled fp32 gradient rows
    loss, _, _, dx = torch.ops.chronicals_hip.ce_logits_fwd_bwd(
        x, lab, int(ignore_index), float(label_smoothing), float(z_loss_weight), _lib.CCE_SMOOTH_UNIFORM,
        _lib.CCE_REDUCTION_MEAN, False, True)
    return loss.view(()), dx.view(logits.shape)


fused_cross_entropy = fused_cross_entropy_triton  # reference :2206-2218 dispatches here on a GPU


# ---------------------------------------------------------------------------
# sequence_packer.py:1660-1717, sequence_packer_v2.py:1058-1113
# ---------------------------------------------------------------------------

def compute_padding_free_loss(
    logits: torch.Tensor,
    labels: torch.Tensor,
    loss_mask=None,
    ignore_index: int = -100,
    reduction: str = "mean",
    label_smoothing: float = 0.0,
) -> torch.Tensor:
    """Cross-entropy of packed sequences (reference sequence_packer.py:1660-1717).

    Per token: torch's label-smoothed cross-entropy
    (1-eps)*(lse - x[label]) + eps*(lse - mean(x)), 0 where the label is
    ``ignore_index``.  Without ``loss_mask``: 'mean' divides the sum by the
    number of labels that are not ``ignore_index`` (at least 1).  With it, each
    token's loss is multiplied by its mask value and 'mean' divides by the
    mask's sum (at least 1).  'none' returns the flat per-token losses.
    """
    red = _reduction_code(reduction)
    x, lab = _rows(logits, labels, "compute_padding_free_loss")
    if loss_mask is None:
        return LogitsCrossEntropyFunction.apply(x, lab, ignore_index, label_smoothing, 0.0,
                                                _lib.CCE_SMOOTH_UNIFORM, red)
    rows = LogitsCrossEntropyFunction.apply(x, lab, ignore_index, label_smoothing, 0.0, _lib.CCE_SMOOTH_UNIFORM,
                                            _lib.CCE_REDUCTION_NONE)
    m = loss_mask.reshape(-1).to(rows.dtype)
    if m.numel() != rows.numel():
        raise RuntimeError(f"loss_mask has {m.numel()} elements, expected {rows.numel()}")
    rows = rows * m
    if red == _lib.CCE_REDUCTION_MEAN:
        return rows.sum() / m.sum().clamp(min=1.0)
    if red == _lib.CCE_REDUCTION_SUM:
        return rows.sum()
    return rows


def compute_packed_loss(
    logits: torch.Tensor,
    labels: torch.Tensor,
    loss_mask=None,
    ignore_index: int = -100,
    reduction: str = "mean",
    label_smoothing: float = 0.0,
) -> torch.Tensor:
    """Cross-entropy of packed sequences (reference sequence_packer_v2.py:1058-1113).

    logits [total_tokens, V] or [batch, seq, V]; the same loss as
    compute_padding_free_loss.
    """
    return compute_padding_free_loss(logits, labels, loss_mask, ignore_index, reduction, label_smoothing)
