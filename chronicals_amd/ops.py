"""torch.library registration of the fused linear-CE entry points.

Two custom operators wrap the C ABI (include/chronicals_cce.h) so the path is
visible to the PyTorch dispatcher and traceable by ``torch.compile``:

  chronicals_hip::cce_fwd(hidden, weight, labels, bias, ignore_index,
                          label_smoothing, z_loss_weight, reduction)
      -> (loss, lse, n_valid)
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
code.  Gradients that are not requested come back as empty
tensors.  Only a HIP-device implementation is registered: CPU tensors raise.
Each fake (meta) implementation gives the output shapes and dtypes without
touching the device.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib

__all__ = ["cce_fwd", "cce_bwd"]


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
            label_smoothing: float, z_loss_weight: float, reduction: int) -> Tuple[Tensor, Tensor, Tensor]:
    _check_operands(hidden, weight, labels, bias)
    hidden, weight = _aligned(hidden), _aligned(weight)
    lib = _lib.load()
    device = hidden.device
    N, d = hidden.shape
    V = weight.shape[0]
    with torch.cuda.device(device):
        ws = torch.empty(_lib.forward_workspace_bytes(N, d, V, reduction), dtype=torch.uint8, device=device)
        loss = torch.empty((N,) if reduction == _lib.CCE_REDUCTION_NONE else (1,), dtype=torch.float32,
                           device=device)
        lse = torch.empty((N,), dtype=torch.float32, device=device)
        n_valid = torch.empty((1,), dtype=torch.int32, device=device)
        _lib.check(lib.cce_forward(
            hidden.data_ptr(), weight.data_ptr(), labels.data_ptr(), int(labels.dtype == torch.int64),
            bias.data_ptr() if bias is not None else None,
            N, d, V, int(ignore_index), float(label_smoothing), float(z_loss_weight), int(reduction),
            loss.data_ptr(), lse.data_ptr(), n_valid.data_ptr(),
            ws.data_ptr(), ws.numel(), _stream(device)))
    return loss, lse, n_valid


@cce_fwd.register_fake
def _cce_fwd_fake(hidden, weight, labels, bias, ignore_index, label_smoothing, z_loss_weight, reduction):
    N = hidden.shape[0]
    loss = hidden.new_empty((N,) if reduction == _lib.CCE_REDUCTION_NONE else (1,), dtype=torch.float32)
    return loss, hidden.new_empty((N,), dtype=torch.float32), hidden.new_empty((1,), dtype=torch.int32)


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
            ws = torch.empty(_lib.backward_workspace_bytes(N, d, V, chunk_size, need_dh, need_dw),
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
