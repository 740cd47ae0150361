"""torch.library registration of the fused linear-CE entry points.

Custom operators wrap the C ABI (include/chronicals_cce.h) so the path is
visible to the PyTorch dispatcher and traceable by ``torch.compile``:

  chronicals_hip::cce_fwd(hidden, weight, labels, bias, ignore_index,
                          label_smoothing, z_loss_weight, smoothing_form,
                          reduction)
      -> (loss, lse, n_valid, target_logit)
  chronicals_hip::cce_bwd(grad_out, hidden, weight, labels, lse, n_valid, bias,
                          ignore_index, label_smoothing, z_loss_weight,
                          reduction, chunk_size, need_dh, need_dw, need_db,
                          dh_f32, dw_f32)
      -> (dh, dw, db)

The reference registers no CE operator (its ``torch.library.Library(
"chronicals", "FRAGMENT")`` at triton_kernels.py:87 holds other ops); these
stand for ``CutCrossEntropyForward.forward`` / ``CutCrossEntropyBackward.
backward`` (cut_cross_entropy.py:567, :703).

Operands: hidden [N, d] and weight [V, d] bf16 and contiguous (a view at an
unaligned storage offset is copied to 16-byte aligned storage); labels [N]
int64 or int32; bias fp32 [V] or None; ``reduction`` is a CCE_REDUCTION_*
code and ``smoothing_form`` a CCE_SMOOTH_* code.  Gradients that are not requested come back as empty
tensors.  Only a HIP-device implementation is registered: CPU tensors raise.
Each fake (meta) implementation gives the output shapes and dtypes without
touching the device.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib

__all__ = ["cce_fwd", "cce_bwd", "ce_logits_fwd", "ce_logits_bwd", "ce_logits_bwd_", "ce_logits_fwd_bwd",
           "ce_logits_fwd_bwd_"]


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _aligned(t: Tensor) -> Tensor:
    """The kernels need 16-byte aligned rows: a view at an unaligned storage
    offset is copied to fresh storage."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _check_operands(hidden: Tensor, weight: Tensor, labels: Tensor, bias: Optional[Tensor]) -> None:
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise RuntimeError(f"cce ops take bf16 hidden and weight, got {hidden.dtype} and {weight.dtype}")
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise RuntimeError(f"cce ops take hidden [N, d] and weight [V, d], got {tuple(hidden.shape)} "
                           f"and {tuple(weight.shape)}")
    if labels.dim() != 1 or labels.shape[0] != hidden.shape[0] or labels.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"cce ops take int64/int32 labels [N], got {labels.dtype} {tuple(labels.shape)}")
    for name, t in (("hidden", hidden), ("weight", weight)):
        if not t.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")
    if bias is not None and (bias.dtype != torch.float32 or bias.shape != (weight.shape[0],)
                             or not bias.is_contiguous()):
        raise RuntimeError("bias must be a contiguous fp32 [V] tensor")


@torch.library.custom_op("chronicals_hip::cce_fwd", mutates_args=(), device_types="cuda")
def cce_fwd(hidden: Tensor, weight: Tensor, labels: Tensor, bias: Optional[Tensor], ignore_index: int,
            label_smoothing: float, z_loss_weight: float, smoothing_form: int, reduction: int,
            lse_rows: int = _lib.CCE_LSE_ALL_ROWS) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    _check_operands(hidden, weight, labels, bias)
    hidden, weight = _aligned(hidden), _aligned(weight)
    lib = _lib.load()
    device = hidden.device
    N, d = hidden.shape
    V = weight.shape[0]
    with torch.cuda.device(device):
        ws = torch.empty(_lib.forward_workspace_bytes(N, d, V, reduction, lse_rows), dtype=torch.uint8,
                         device=device)
        loss = torch.empty((N,) if reduction == _lib.CCE_REDUCTION_NONE else (1,), dtype=torch.float32,
                           device=device)
        lse = torch.empty((N,), dtype=torch.float32, device=device)
        target = torch.empty((N,), dtype=torch.float32, device=device)
        n_valid = torch.empty((1,), dtype=torch.int32, device=device)
        _lib.check(lib.cce_forward(
            hidden.data_ptr(), weight.data_ptr(), labels.data_ptr(), int(labels.dtype == torch.int64),
            bias.data_ptr() if bias is not None else None,
            N, d, V, int(ignore_index), float(label_smoothing), float(z_loss_weight), int(smoothing_form),
            int(reduction), int(lse_rows), loss.data_ptr(), lse.data_ptr(), target.data_ptr(), n_valid.data_ptr(),
            ws.data_ptr(), ws.numel(), _stream(device)))
    return loss, lse, n_valid, target


@cce_fwd.register_fake
def _cce_fwd_fake(hidden, weight, labels, bias, ignore_index, label_smoothing, z_loss_weight, smoothing_form,
                  reduction, lse_rows=_lib.CCE_LSE_ALL_ROWS):
    N = hidden.shape[0]
    loss = hidden.new_empty((N,) if reduction == _lib.CCE_REDUCTION_NONE else (1,), dtype=torch.float32)
    return (loss, hidden.new_empty((N,), dtype=torch.float32), hidden.new_empty((1,), dtype=torch.int32),
            hidden.new_empty((N,), dtype=torch.float32))


@torch.library.custom_op("chronicals_hip::cce_bwd", mutates_args=(), device_types="cuda")
def cce_bwd(grad_out: Tensor, hidden: Tensor, weight: Tensor, labels: Tensor, lse: Tensor, n_valid: Tensor,
            bias: Optional[Tensor], ignore_index: int, label_smoothing: float, z_loss_weight: float,
            reduction: int, chunk_size: int, need_dh: bool, need_dw: bool, need_db: bool, dh_f32: bool,
            dw_f32: bool) -> Tuple[Tensor, Tensor, Tensor]:
    _check_operands(hidden, weight, labels, bias)
    if need_db and bias is None:
        raise RuntimeError("need_db requires a bias")
    hidden, weight = _aligned(hidden), _aligned(weight)
    lib = _lib.load()
    device = hidden.device
    N, d = hidden.shape
    V = weight.shape[0]
    g = grad_out.detach().to(torch.float32).reshape(-1).contiguous()
    with torch.cuda.device(device):
        dh = torch.empty((N, d) if need_dh else (0,), dtype=torch.float32 if dh_f32 else torch.bfloat16,
                         device=device)
        dw = torch.empty((V, d) if need_dw else (0,), dtype=torch.float32 if dw_f32 else torch.bfloat16,
                         device=device)
        db = torch.empty((V,) if need_db else (0,), dtype=torch.float32, device=device)
        if need_dh or need_dw or need_db:
            ws = torch.empty(_lib.backward_workspace_bytes(N, d, V, chunk_size, need_dh, need_dw, dh_f32, dw_f32),
                             dtype=torch.uint8, device=device)
            _lib.check(lib.cce_backward(
                g.data_ptr(), hidden.data_ptr(), weight.data_ptr(), labels.data_ptr(),
                int(labels.dtype == torch.int64), bias.data_ptr() if bias is not None else None,
                lse.data_ptr(), n_valid.data_ptr(), N, d, V, int(ignore_index), float(label_smoothing),
                float(z_loss_weight), int(reduction), int(chunk_size),
                dh.data_ptr() if need_dh else None, _lib.CCE_DTYPE_F32 if dh_f32 else _lib.CCE_DTYPE_BF16,
                dw.data_ptr() if need_dw else None, _lib.CCE_DTYPE_F32 if dw_f32 else _lib.CCE_DTYPE_BF16,
                db.data_ptr() if need_db else None,
                ws.data_ptr(), ws.numel(), _stream(device)))
    return dh, dw, db


@cce_bwd.register_fake
def _cce_bwd_fake(grad_out, hidden, weight, labels, lse, n_valid, bias, ignore_index, label_smoothing,
                  z_loss_weight, reduction, chunk_size, need_dh, need_dw, need_db, dh_f32, dw_f32):
    N, d = hidden.shape
    V = weight.shape[0]
    dh = hidden.new_empty((N, d) if need_dh else (0,), dtype=torch.float32 if dh_f32 else torch.bfloat16)
    dw = hidden.new_empty((V, d) if need_dw else (0,), dtype=torch.float32 if dw_f32 else torch.bfloat16)
    db = hidden.new_empty((V,) if need_db else (0,), dtype=torch.float32)
    return dh, dw, db


# ---------------------------------------------------------------------------
# Cross-entropy over existing logits (cce_logits_forward / cce_logits_backward)
#
#   chronicals_hip::ce_logits_fwd(logits, labels, ignore_index, label_smoothing,
#                                 z_loss_weight, smoothing_form, reduction)
#                                 -> (loss, lse, n_valid)
#   chronicals_hip::ce_logits_bwd(grad_out, logits, labels, lse, n_valid,
#                                 ignore_index, label_smoothing, z_loss_weight,
#                                 smoothing_form, reduction, f32_grad) -> grad_logits
#   chronicals_hip::ce_logits_bwd_(... same ...)  overwrites logits with the gradient
#
# logits [N, V] bf16 / fp16 / fp32 with a contiguous last dimension (any row
# stride).  ce_logits_bwd returns a contiguous [N, V] tensor of the logits'
# dtype (fp32 when f32_grad).
# ---------------------------------------------------------------------------

_LOGITS_DTYPES = {torch.bfloat16: _lib.CCE_DTYPE_BF16, torch.float16: _lib.CCE_DTYPE_F16,
                  torch.float32: _lib.CCE_DTYPE_F32}


def _check_logits(logits: Tensor, labels: Tensor) -> None:
    if logits.dtype not in _LOGITS_DTYPES:
        raise RuntimeError(f"logits dtype {logits.dtype} not supported (bf16, fp16, fp32)")
    if logits.dim() != 2 or (logits.shape[1] > 1 and logits.stride(1) != 1):
        raise RuntimeError(f"ce_logits ops take [N, V] logits with a contiguous last dimension, got "
                           f"shape {tuple(logits.shape)} strides {logits.stride()}")
    if labels.dim() != 1 or labels.shape[0] != logits.shape[0] or labels.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"ce_logits ops take int64/int32 labels [N], got {labels.dtype} {tuple(labels.shape)}")
    if not labels.is_contiguous():
        raise RuntimeError("labels must be contiguous")


def _row_stride(t: Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


@torch.library.custom_op("chronicals_hip::ce_logits_fwd", mutates_args=(), device_types="cuda")
def ce_logits_fwd(logits: Tensor, labels: Tensor, ignore_index: int, label_smoothing: float, z_loss_weight: float,
                  smoothing_form: int, reduction: int) -> Tuple[Tensor, Tensor, Tensor]:
    _check_logits(logits, labels)
    lib = _lib.load()
    device = logits.device
    N, V = logits.shape
    with torch.cuda.device(device):
        ws = torch.empty(_lib.logits_forward_workspace_bytes(N, V, reduction), dtype=torch.uint8, device=device)
        loss = torch.empty((N,) if reduction == _lib.CCE_REDUCTION_NONE else (1,), dtype=torch.float32,
                           device=device)
        lse = torch.empty((N,), dtype=torch.float32, device=device)
        n_valid = torch.empty((1,), dtype=torch.int32, device=device)
        _lib.check(lib.cce_logits_forward(
            logits.data_ptr(), _LOGITS_DTYPES[logits.dtype], _row_stride(logits), labels.data_ptr(),
            int(labels.dtype == torch.int64), N, V, int(ignore_index), float(label_smoothing), float(z_loss_weight),
            int(smoothing_form), int(reduction), loss.data_ptr(), lse.data_ptr(), n_valid.data_ptr(), ws.data_ptr(),
            ws.numel(), _stream(device)))
    return loss, lse, n_valid


@ce_logits_fwd.register_fake
def _ce_logits_fwd_fake(logits, labels, ignore_index, label_smoothing, z_loss_weight, smoothing_form, reduction):
    N = logits.shape[0]
    loss = logits.new_empty((N,) if reduction == _lib.CCE_REDUCTION_NONE else (1,), dtype=torch.float32)
    return loss, logits.new_empty((N,), dtype=torch.float32), logits.new_empty((1,), dtype=torch.int32)


def _logits_backward(grad_out: Tensor, logits: Tensor, labels: Tensor, lse: Tensor, n_valid: Tensor,
                     ignore_index: int, label_smoothing: float, z_loss_weight: float, smoothing_form: int,
                     reduction: int, out: Tensor) -> None:
    _check_logits(logits, labels)
    N, V = logits.shape
    if N == 0:
        return
    lib = _lib.load()
    device = logits.device
    g = grad_out.detach().to(torch.float32).reshape(-1).contiguous()
    with torch.cuda.device(device):
        _lib.check(lib.cce_logits_backward(
            g.data_ptr(), logits.data_ptr(), _LOGITS_DTYPES[logits.dtype], _row_stride(logits), labels.data_ptr(),
            int(labels.dtype == torch.int64), lse.data_ptr(), n_valid.data_ptr(), N, V, int(ignore_index),
            float(label_smoothing), float(z_loss_weight), int(smoothing_form), int(reduction), out.data_ptr(),
            _LOGITS_DTYPES[out.dtype], _row_stride(out), _stream(device)))


@torch.library.custom_op("chronicals_hip::ce_logits_bwd", mutates_args=(), device_types="cuda")
def ce_logits_bwd(grad_out: Tensor, logits: Tensor, labels: Tensor, lse: Tensor, n_valid: Tensor, ignore_index: int,
                  label_smoothing: float, z_loss_weight: float, smoothing_form: int, reduction: int,
                  f32_grad: bool) -> Tensor:
    dx = torch.empty(tuple(logits.shape), dtype=torch.float32 if f32_grad else logits.dtype, device=logits.device)
    _logits_backward(grad_out, logits, labels, lse, n_valid, ignore_index, label_smoothing, z_loss_weight,
                     smoothing_form, reduction, dx)
    return dx


@ce_logits_bwd.register_fake
def _ce_logits_bwd_fake(grad_out, logits, labels, lse, n_valid, ignore_index, label_smoothing, z_loss_weight,
                        smoothing_form, reduction, f32_grad):
    return logits.new_empty(tuple(logits.shape), dtype=torch.float32 if f32_grad else logits.dtype)


@torch.library.custom_op("chronicals_hip::ce_logits_bwd_", mutates_args=("logits",), device_types="cuda")
def ce_logits_bwd_(grad_out: Tensor, logits: Tensor, labels: Tensor, lse: Tensor, n_valid: Tensor,
                   ignore_index: int, label_smoothing: float, z_loss_weight: float, smoothing_form: int,
                   reduction: int) -> None:
    _logits_backward(grad_out, logits, labels, lse, n_valid, ignore_index, label_smoothing, z_loss_weight,
                     smoothing_form, reduction, logits)


@ce_logits_bwd_.register_fake
def _ce_logits_bwd__fake(grad_out, logits, labels, lse, n_valid, ignore_index, label_smoothing, z_loss_weight,
                         smoothing_form, reduction):
    return None


# ---------------------------------------------------------------------------
# Loss and gradient in one kernel (cce_logits_forward_backward)
#
#   chronicals_hip::ce_logits_fwd_bwd(logits, labels, ignore_index, label_smoothing,
#                                     z_loss_weight, smoothing_form, reduction,
#                                     grad_mean, f32_grad) -> (loss, lse, n_valid, grad_logits)
#   chronicals_hip::ce_logits_fwd_bwd_(...without f32_grad...) -> (loss, lse, n_valid),
#                                     the gradient written over the logits
# ---------------------------------------------------------------------------

def _logits_forward_backward(logits: Tensor, labels: Tensor, ignore_index: int, label_smoothing: float,
                             z_loss_weight: float, smoothing_form: int, reduction: int, grad_mean: bool,
                             out: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    _check_logits(logits, labels)
    lib = _lib.load()
    device = logits.device
    N, V = logits.shape
    with torch.cuda.device(device):
        ws = torch.empty(_lib.logits_forward_workspace_bytes(N, V, reduction), dtype=torch.uint8, device=device)
        loss = torch.empty((N,) if reduction == _lib.CCE_REDUCTION_NONE else (1,), dtype=torch.float32,
                           device=device)
        lse = torch.empty((N,), dtype=torch.float32, device=device)
        n_valid = torch.empty((1,), dtype=torch.int32, device=device)
        _lib.check(lib.cce_logits_forward_backward(
            logits.data_ptr(), _LOGITS_DTYPES[logits.dtype], _row_stride(logits), labels.data_ptr(),
            int(labels.dtype == torch.int64), N, V, int(ignore_index), float(label_smoothing), float(z_loss_weight),
            int(smoothing_form), int(reduction), int(bool(grad_mean)), loss.data_ptr(), lse.data_ptr(),
            n_valid.data_ptr(), out.data_ptr(), _LOGITS_DTYPES[out.dtype], _row_stride(out), ws.data_ptr(),
            ws.numel(), _stream(device)))
    return loss, lse, n_valid


@torch.library.custom_op("chronicals_hip::ce_logits_fwd_bwd", mutates_args=(), device_types="cuda")
def ce_logits_fwd_bwd(logits: Tensor, labels: Tensor, ignore_index: int, label_smoothing: float, z_loss_weight: float,
                      smoothing_form: int, reduction: int, grad_mean: bool,
                      f32_grad: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    dx = torch.empty(tuple(logits.shape), dtype=torch.float32 if f32_grad else logits.dtype, device=logits.device)
    loss, lse, n_valid = _logits_forward_backward(logits, labels, ignore_index, label_smoothing, z_loss_weight,
                                                  smoothing_form, reduction, grad_mean, dx)
    return loss, lse, n_valid, dx


@ce_logits_fwd_bwd.register_fake
def _ce_logits_fwd_bwd_fake(logits, labels, ignore_index, label_smoothing, z_loss_weight, smoothing_form, reduction,
                            grad_mean, f32_grad):
    loss, lse, nv = _ce_logits_fwd_fake(logits, labels, ignore_index, label_smoothing, z_loss_weight, smoothing_form,
                                        reduction)
    return loss, lse, nv, logits.new_empty(tuple(logits.shape), dtype=torch.float32 if f32_grad else logits.dtype)


@torch.library.custom_op("chronicals_hip::ce_logits_fwd_bwd_", mutates_args=("logits",), device_types="cuda")
def ce_logits_fwd_bwd_(logits: Tensor, labels: Tensor, ignore_index: int, label_smoothing: float,
                       z_loss_weight: float, smoothing_form: int, reduction: int,
                       grad_mean: bool) -> Tuple[Tensor, Tensor, Tensor]:
    return _logits_forward_backward(logits, labels, ignore_index, label_smoothing, z_loss_weight, smoothing_form,
                                    reduction, grad_mean, logits)


@ce_logits_fwd_bwd_.register_fake
def _ce_logits_fwd_bwd__fake(logits, labels, ignore_index, label_smoothing, z_loss_weight, smoothing_form, reduction,
                             grad_mean):
    return _ce_logits_fwd_fake(logits, labels, ignore_index, label_smoothing, z_loss_weight, smoothing_form,
                               reduction)
