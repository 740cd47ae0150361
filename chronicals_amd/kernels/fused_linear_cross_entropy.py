"""The reference's sibling fused linear cross-entropy APIs, on the same HIP kernels.

``chronicals.kernels.triton_kernels`` exposes two more front ends to the
fused lm_head projection + cross-entropy beside ``cut_cross_entropy``; both
run here on ``cce_forward`` / ``cce_backward`` (include/chronicals_cce.h):

  fused_linear_cross_entropy_forward, fused_linear_cross_entropy,
  FusedLinearCrossEntropyFunction, fused_linear_cross_entropy_autograd,
  FusedLinearCrossEntropyLoss (alias ChunkedCrossEntropyLoss)
      reference triton_kernels.py:2308-2817.  Loss with eps*log(V) label
      smoothing, z-loss default 1e-4, reductions mean / sum / none; returns
      (loss, z_loss).  Gradient P - (1-eps)*onehot - eps/V + 2z*lse*P
      (:2562-2616).
  triton_fused_linear_cross_entropy_forward, TritonFusedLinearCrossEntropyFunction,
  triton_fused_linear_cross_entropy, TritonFusedLinearCrossEntropyLoss
  (alias LigerFusedLinearCrossEntropyLoss)
      reference triton_kernels.py:3147-3419.  The uniform-target label
      smoothing loss of _liger_ce_kernel (:2914-2956), same gradient.
  chunked_cross_entropy
      reference triton_kernels.py:2659-2731: the legacy logits-in loss (mean
      over valid rows of the eps*log(V) loss + z * mean lse^2), on the row
      kernels of ``logits_cross_entropy``.

Deliberate differences from the reference:
  * Tensors must live on a HIP device; hidden and weight are computed in
    bf16 with fp32 accumulation, gradients come back in the input dtypes.
  * ``z_loss`` (the monitoring output of the (loss, z_loss) pairs) carries
    no gradient; ``FusedLinearCrossEntropyFunction``'s backward ignores it in
    the reference too (:2544-2616).
  * ``TritonFusedLinearCrossEntropyFunction`` computes the gradients in
    backward with grad_output folded in (the reference computes them in
    forward and rescales), and 'none' works in backward (the reference's
    rescaling compares a tensor with 1.0 there, :3294).
  * ``chunked_cross_entropy`` returns 0 when every label is ignored (the
    reference's mean of an empty selection is NaN).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .. import _lib
from .cut_cross_entropy import _backward_raw, _forward_raw, _LinearCE, _reduction_code
from .logits_cross_entropy import LogitsCrossEntropyFunction, _rows

DEFAULT_CHUNK_SIZE = 8192  # reference triton_kernels.py:2297

__all__ = [
    "DEFAULT_CHUNK_SIZE",
    "fused_linear_cross_entropy_forward",
    "fused_linear_cross_entropy",
    "FusedLinearCrossEntropyFunction",
    "fused_linear_cross_entropy_autograd",
    "FusedLinearCrossEntropyLoss",
    "ChunkedCrossEntropyLoss",
    "chunked_cross_entropy",
    "triton_fused_linear_cross_entropy_forward",
    "TritonFusedLinearCrossEntropyFunction",
    "triton_fused_linear_cross_entropy",
    "TritonFusedLinearCrossEntropyLoss",
    "LigerFusedLinearCrossEntropyLoss",
]


def _z_loss(lse: torch.Tensor, labels: torch.Tensor, ignore_index: int, z: float, red: int) -> torch.Tensor:
    """z * lse^2 over the valid rows, reduced like the loss (monitoring only)."""
    valid = (labels.reshape(-1) != ignore_index).to(lse.dtype)
    rows = z * lse * lse * valid
    if red == _lib.CCE_REDUCTION_MEAN:
        return rows.sum() / valid.sum().clamp(min=1)
    if red == _lib.CCE_REDUCTION_SUM:
        return rows.sum()
    return rows.view(labels.shape)


# ---------------------------------------------------------------------------
# triton_kernels.py:2308-2817
# ---------------------------------------------------------------------------

def fused_linear_cross_entropy_forward(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    labels: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    chunk_size: int = DEFAULT_CHUNK_SIZE,
    ignore_index: int = -100,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(logsumexp [N], target_logit [N], valid_mask [N]) without logits (reference :2308-2396).

    lse = log(sum_v exp(hidden . weight[v] + bias[v]) + 1e-10); the target
    logit is 0 for ignored rows and for labels outside [0, V).  No gradient.
    """
    del chunk_size
    with torch.no_grad():
        _, lse, _, _, _, lab, _, target = _forward_raw(hidden, weight, labels, bias, ignore_index, 0.0, 0.0,
                                                       _lib.CCE_REDUCTION_MEAN)
    return lse, target, lab != ignore_index


def fused_linear_cross_entropy(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    labels: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    label_smoothing: float = 0.0,
    z_loss_weight: float = 1e-4,
    ignore_index: int = -100,
    chunk_size: int = DEFAULT_CHUNK_SIZE,
    reduction: str = "mean",
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(loss, z_loss) of the fused linear cross-entropy (reference :2398-2493).

    loss per valid row (1-eps)*(lse - target) + eps*log(V) + z*lse^2, reduced
    ('mean': / max(n_valid, 1)); z_loss is the z*lse^2 part, reduced the same
    way.  ``loss`` is differentiable in hidden, weight and bias.
    """
    red = _reduction_code(reduction)
    loss, lse = _LinearCE.apply(hidden, weight, labels, bias, chunk_size, ignore_index, label_smoothing,
                                z_loss_weight, red, _lib.CCE_SMOOTH_LOGV)
    return loss, _z_loss(lse.detach(), labels, ignore_index, z_loss_weight, red)


class FusedLinearCrossEntropyFunction(torch.autograd.Function):
    """Autograd with the reference's argument order (triton_kernels.py:2496-2633).

    apply(hidden, weight, bias, labels, label_smoothing, z_loss_weight,
          ignore_index, chunk_size) -> (loss, z_loss), 'mean' reduction.
    """

    @staticmethod
    def forward(ctx, hidden, weight, bias, labels, label_smoothing, z_loss_weight, ignore_index, chunk_size):
        red = _lib.CCE_REDUCTION_MEAN
        loss, lse, n_valid, h2, w2, lab, b32, _ = _forward_raw(hidden, weight, labels, bias, ignore_index,
                                                            label_smoothing, z_loss_weight, red,
                                                            lse_rows=_lib.CCE_LSE_LABELLED_ROWS)
        ctx.save_for_backward(h2, w2, lab, lse, n_valid, b32)
        ctx.cfg = (int(chunk_size), int(ignore_index), float(label_smoothing), float(z_loss_weight), red)
        ctx.shapes = (hidden.shape, hidden.dtype, weight.dtype, None if bias is None else bias.dtype)
        z_loss = _z_loss(lse, labels, ignore_index, z_loss_weight, red)
        ctx.mark_non_differentiable(z_loss)
        return loss.view(()), z_loss

    @staticmethod
    def backward(ctx, grad_loss, grad_z_loss):
        del grad_z_loss
        dh, dw, db = _backward_raw(ctx, grad_loss, ctx.needs_input_grad[0], ctx.needs_input_grad[1],
                                   ctx.needs_input_grad[2])
        return dh, dw, db, None, None, None, None, None


def fused_linear_cross_entropy_autograd(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    labels: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    label_smoothing: float = 0.0,
    z_loss_weight: float = 1e-4,
    ignore_index: int = -100,
    chunk_size: int = DEFAULT_CHUNK_SIZE,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """FusedLinearCrossEntropyFunction.apply in the reference's keyword order (:2636-2656)."""
    return FusedLinearCrossEntropyFunction.apply(hidden, weight, bias, labels, label_smoothing, z_loss_weight,
                                                 ignore_index, chunk_size)


class FusedLinearCrossEntropyLoss(nn.Module):
    """Module form (reference :2734-2814): forward(hidden, weight, bias, labels) -> (loss, z_loss)."""

    def __init__(self, chunk_size: int = DEFAULT_CHUNK_SIZE, label_smoothing: float = 0.0,
                 z_loss_weight: float = 1e-4, ignore_index: int = -100):
        super().__init__()
        self.chunk_size = chunk_size
        self.label_smoothing = label_smoothing
        self.z_loss_weight = z_loss_weight
        self.ignore_index = ignore_index

    def forward(self, hidden: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                labels: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        return fused_linear_cross_entropy_autograd(hidden, weight, labels, bias, self.label_smoothing,
                                                   self.z_loss_weight, self.ignore_index, self.chunk_size)

    def extra_repr(self) -> str:
        return (f"chunk_size={self.chunk_size}, label_smoothing={self.label_smoothing}, "
                f"z_loss_weight={self.z_loss_weight}, ignore_index={self.ignore_index}")


ChunkedCrossEntropyLoss = FusedLinearCrossEntropyLoss  # reference :2817


def chunked_cross_entropy(
    logits: torch.Tensor,
    labels: torch.Tensor,
    chunk_size: int = 8192,
    label_smoothing: float = 0.0,
    z_loss_weight: float = 1e-4,
    ignore_index: int = -100,
) -> torch.Tensor:
    """Legacy logits-in loss (reference :2659-2731): mean over valid rows of
    (1-eps)*(lse - logit[label]) + eps*log(V), plus z * mean lse^2."""
    del chunk_size
    x, lab = _rows(logits, labels, "chunked_cross_entropy")
    return LogitsCrossEntropyFunction.apply(x, lab, ignore_index, label_smoothing, z_loss_weight,
                                            _lib.CCE_SMOOTH_LOGV, _lib.CCE_REDUCTION_MEAN)


# ---------------------------------------------------------------------------
# triton_kernels.py:3147-3419
# ---------------------------------------------------------------------------

def triton_fused_linear_cross_entropy_forward(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    target: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    ignore_index: int = -100,
    lse_square_scale: float = 0.0,
    label_smoothing: float = 0.0,
    reduction: str = "mean",
    chunk_size: int = 8192,
) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
    """(loss, grad_hidden, grad_weight, grad_bias), gradients computed now (reference :3147-3276).

    Uniform-target smoothing: per valid row (1-eps)*(lse - target) +
    eps*(lse - mean_v logits) + s*lse^2.  Gradients of the 'mean' loss are
    divided by n_valid; 'sum' and 'none' gradients are those of the sum.
    grad_weight is None when weight does not require grad, grad_bias when
    there is no bias or it does not require grad.
    """
    red = _reduction_code(reduction)
    need_dw = bool(weight.requires_grad)
    need_db = bias is not None and bool(bias.requires_grad)
    with torch.no_grad():
        loss, lse, n_valid, h2, w2, lab, b32, _ = _forward_raw(hidden, weight, target, bias, ignore_index,
                                                            label_smoothing, lse_square_scale, red,
                                                            _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_LSE_LABELLED_ROWS)
        gred = _lib.CCE_REDUCTION_SUM if red == _lib.CCE_REDUCTION_NONE else red
        one = torch.ones((1,), dtype=torch.float32, device=h2.device)
        dh, dw, db = torch.ops.chronicals_hip.cce_bwd(
            one, h2, w2, lab, lse, n_valid, b32, int(ignore_index), float(label_smoothing),
            float(lse_square_scale), gred, int(chunk_size), True, need_dw, need_db,
            hidden.dtype != torch.bfloat16, weight.dtype != torch.bfloat16)
    loss = loss.view(target.shape) if red == _lib.CCE_REDUCTION_NONE else loss.view(())
    dh = dh.view(hidden.shape).to(hidden.dtype)
    dw = dw.to(weight.dtype) if need_dw else None
    db = db.to(bias.dtype) if need_db else None
    return loss, dh, dw, db


class TritonFusedLinearCrossEntropyFunction(torch.autograd.Function):
    """Autograd with the reference's arguments (triton_kernels.py:3279-3315).

    apply(hidden, weight, target, bias=None, ignore_index=-100, lse_scale=0.0,
          label_smoothing=0.0, reduction='mean', chunk_size=8192) -> loss
    """

    @staticmethod
    def forward(ctx, hidden, weight, target, bias=None, ignore_index=-100, lse_scale=0.0, label_smoothing=0.0,
                reduction="mean", chunk_size=8192):
        red = _reduction_code(reduction)
        loss, lse, n_valid, h2, w2, lab, b32, _ = _forward_raw(hidden, weight, target, bias, ignore_index,
                                                            label_smoothing, lse_scale, red,
                                                            _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_LSE_LABELLED_ROWS)
        ctx.save_for_backward(h2, w2, lab, lse, n_valid, b32)
        ctx.cfg = (int(chunk_size), int(ignore_index), float(label_smoothing), float(lse_scale), red)
        ctx.shapes = (hidden.shape, hidden.dtype, weight.dtype, None if bias is None else bias.dtype)
        return loss.view(target.shape) if red == _lib.CCE_REDUCTION_NONE else loss.view(())

    @staticmethod
    def backward(ctx, grad_output):
        dh, dw, db = _backward_raw(ctx, grad_output, ctx.needs_input_grad[0], ctx.needs_input_grad[1],
                                   ctx.needs_input_grad[3])
        return dh, dw, None, db, None, None, None, None, None


def triton_fused_linear_cross_entropy(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    target: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    ignore_index: int = -100,
    lse_square_scale: float = 0.0,
    label_smoothing: float = 0.0,
    reduction: str = "mean",
    chunk_size: int = 8192,
) -> torch.Tensor:
    """Differentiable uniform-smoothing fused linear cross-entropy (reference :3318-3370)."""
    return TritonFusedLinearCrossEntropyFunction.apply(hidden, weight, target, bias, ignore_index, lse_square_scale,
                                                       label_smoothing, reduction, chunk_size)


class TritonFusedLinearCrossEntropyLoss(nn.Module):
    """Module form (reference :3373-3416): forward(hidden, weight, target, bias=None) -> loss."""

    def __init__(self, chunk_size: int = 8192, ignore_index: int = -100, lse_square_scale: float = 0.0,
                 label_smoothing: float = 0.0, reduction: str = "mean"):
        super().__init__()
        _reduction_code(reduction)
        self.chunk_size = chunk_size
        self.ignore_index = ignore_index
        self.lse_square_scale = lse_square_scale
        self.label_smoothing = label_smoothing
        self.reduction = reduction

    def forward(self, hidden: torch.Tensor, weight: torch.Tensor, target: torch.Tensor,
                bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        return triton_fused_linear_cross_entropy(hidden, weight, target, bias, self.ignore_index,
                                                 self.lse_square_scale, self.label_smoothing, self.reduction,
                                                 self.chunk_size)

    def extra_repr(self) -> str:
        return (f"chunk_size={self.chunk_size}, ignore_index={self.ignore_index}, "
                f"lse_scale={self.lse_square_scale}, label_smoothing={self.label_smoothing}")


LigerFusedLinearCrossEntropyLoss = TritonFusedLinearCrossEntropyLoss  # reference :3419
