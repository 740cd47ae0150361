"""Shared helpers for the CCE tests: seeded inputs, tolerances, references.

Input recipes follow the five BASELINE configurations (C1..C5): hidden ~
N(0,1), W ~ N(0, 0.02), labels uniform (C3: Zipf(1.1)), a fraction of rows
set to ignore_index = -100 (C4: the first token of every packed sequence).
Generation order is hidden, W, labels, ignore mask from one seeded
torch.Generator, so a case regenerates identically on any host.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

IGNORE = -100

# Tolerances of the contract: loss within 1e-3 relative; gradients with max
# abs error <= 2e-2 * max|reference grad| and cosine >= 0.9999.
LOSS_RTOL = 1e-3
GRAD_MAXABS_FRAC = 2e-2
GRAD_COS_MIN = 0.9999


@dataclass(frozen=True)
class Config:
    name: str
    N: int
    d: int
    V: int
    dtype: torch.dtype
    ignore_frac: float
    labels: str = "uniform"   # uniform | zipf | packed
    reduction: str = "mean"


CONFIGS = {
    "C1": Config("C1", 256, 768, 50257, torch.float32, 0.10),
    "C2": Config("C2", 16384, 896, 151936, torch.bfloat16, 0.05),
    "C3": Config("C3", 8192, 4096, 128256, torch.bfloat16, 0.02, labels="zipf"),
    "C4": Config("C4", 32768, 2048, 151936, torch.bfloat16, 0.0, labels="packed"),
    "C5": Config("C5", 65536, 3584, 152064, torch.bfloat16, 0.05),
}


def zipf_labels(n: int, V: int, s: float, gen: torch.Generator) -> torch.Tensor:
    """Inverse-CDF sampling of p(k) proportional to (k+1)^-s over [0, V), on the generator's device."""
    dev = gen.device
    k = torch.arange(V, dtype=torch.float64, device=dev)
    p = (k + 1.0) ** (-s)
    cdf = torch.cumsum(p, 0)
    cdf = cdf / cdf[-1]
    u = torch.rand(n, generator=gen, dtype=torch.float64, device=dev)
    idx = torch.searchsorted(cdf, u).clamp_(max=V - 1)
    return idx.to(torch.int64)


def packed_first_token_mask(n: int, gen: torch.Generator, lo: int = 64, hi: int = 2048) -> torch.Tensor:
    """True at the first token of each packed sequence (lengths U{lo..hi}, last one truncated to fill n)."""
    mask = torch.zeros(n, dtype=torch.bool)
    pos = 0
    while pos < n:
        mask[pos] = True
        pos += int(torch.randint(lo, hi + 1, (1,), generator=gen, device=gen.device).item())
    return mask.to(gen.device)


def make_inputs(cfg: Config, seed: int = 0, N: Optional[int] = None, device="cpu", gen_device="cpu"):
    """(hidden [N,d], weight [V,d], labels [N] int64) for a config, optionally with fewer rows.

    One torch.Generator seeded with `seed` draws, in this order: hidden ~
    N(0,1) [N,d], W ~ N(0,0.02) [V,d] (fp32, then cast to the config's
    dtype), the labels (uniform over [0,V), or Zipf(1.1) for C3), then the
    ignore mask (C4: the first token of each packed sequence; the others:
    each row with probability ignore_frac).  With gen_device="cpu" (the
    default) the values are the same on any host; gen_device="cuda" draws the
    same recipe with a device generator (fast at full size; other values).
    """
    n = cfg.N if N is None else N
    g = torch.Generator(device=gen_device).manual_seed(seed)
    hidden = torch.randn(n, cfg.d, generator=g, device=gen_device, dtype=torch.float32)
    weight = torch.randn(cfg.V, cfg.d, generator=g, device=gen_device, dtype=torch.float32) * 0.02
    if cfg.labels == "zipf":
        labels = zipf_labels(n, cfg.V, 1.1, g)
    else:
        labels = torch.randint(0, cfg.V, (n,), generator=g, dtype=torch.int64, device=gen_device)
    if cfg.labels == "packed":
        labels[packed_first_token_mask(n, g)] = IGNORE
    if cfg.ignore_frac > 0:
        drop = torch.rand(n, generator=g, device=gen_device) < cfg.ignore_frac
        labels[drop] = IGNORE
    hidden = hidden.to(cfg.dtype).to(device)
    weight = weight.to(cfg.dtype).to(device)
    return hidden, weight, labels.to(device)


def bf16_exact(x: torch.Tensor) -> torch.Tensor:
    """fp32 copy of x rounded to bf16 (what the kernel consumes)."""
    return x.detach().to(torch.bfloat16).to(torch.float32)


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    if na == 0 or nb == 0:
        return 0.0
    return float(a @ b / (na * nb))


def grad_report(got, ref) -> dict:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    err = float(np.abs(got - ref).max()) if ref.size else 0.0
    return {"max_abs_err": err, "max_ref": scale, "frac": err / scale if scale > 0 else err,
            "cos": cosine(got, ref)}


def assert_grad_close(got, ref, what: str):
    r = grad_report(got, ref)
    if r["max_ref"] == 0.0:
        assert r["max_abs_err"] <= 1e-6, f"{what}: expected zeros, {r}"
        return
    assert r["frac"] <= GRAD_MAXABS_FRAC, f"{what}: max abs err too large {r}"
    assert r["cos"] >= GRAD_COS_MIN, f"{what}: cosine too small {r}"


def assert_loss_close(got, ref, what: str = "loss", rtol: float = LOSS_RTOL, atol: float = 1e-6):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    tol = atol + rtol * np.abs(ref)
    assert np.all(err <= tol), f"{what}: max err {err.max()} (ref max {np.abs(ref).max()})"


def torch_reference(hidden, weight, labels, bias=None, ignore_index=IGNORE, label_smoothing=0.0, z_loss_weight=0.0,
                    reduction="mean", dtype=torch.float64, grad_output=None):
    """Materialised-logits reference with autograd (any device, given dtype).

    loss_row = (1-eps)*CE + eps*log(V) + z*lse^2 (reference
    cut_cross_entropy.py:674-683).  Its gradient is computed by autograd of
    (1-eps)*CE + eps*(lse - mean logits) + z*lse^2, i.e. torch's own
    label-smoothed cross-entropy, whose logit gradient is the reference's
    P - (1-eps)*onehot - eps/V + 2z*lse*P (:773-789).
    """
    h = hidden.detach().to(dtype).reshape(-1, hidden.shape[-1]).requires_grad_(True)
    w = weight.detach().to(dtype).requires_grad_(True)
    b = None if bias is None else bias.detach().to(dtype).requires_grad_(True)
    lab = labels.reshape(-1)
    V = w.shape[0]
    logits = h @ w.t()
    if b is not None:
        logits = logits + b
    valid = lab != ignore_index
    in_range = valid & (lab >= 0) & (lab < V)
    lse = torch.logsumexp(logits, dim=-1)
    safe = torch.where(in_range, lab, torch.zeros_like(lab))
    tgt = logits.gather(1, safe[:, None])[:, 0] * in_range.to(dtype)
    ce = lse - tgt
    smooth_grad_term = lse - logits.mean(dim=-1)
    row_grad = (1 - label_smoothing) * ce + label_smoothing * smooth_grad_term + z_loss_weight * lse * lse
    row_val = (1 - label_smoothing) * ce + label_smoothing * math.log(V) + z_loss_weight * lse * lse
    vmask = valid.to(dtype)
    n_valid = max(int(valid.sum().item()), 1)
    if reduction == "mean":
        obj = (row_grad * vmask).sum() / n_valid
        val = (row_val * vmask).sum() / n_valid
    elif reduction == "sum":
        obj = (row_grad * vmask).sum()
        val = (row_val * vmask).sum()
    else:
        go = torch.ones_like(lse) if grad_output is None else grad_output.to(dtype).reshape(-1)
        obj = (row_grad * vmask * go).sum()
        val = row_val * vmask
    if grad_output is not None and reduction != "none":
        obj = obj * float(grad_output)
    obj.backward()
    return {
        "loss": val.detach(),
        "lse": lse.detach(),
        "dh": h.grad.detach().reshape(hidden.shape),
        "dw": w.grad.detach(),
        "db": None if b is None else b.grad.detach(),
    }


def torch_reference_rows(hidden, weight, labels, ignore_index=IGNORE, dtype=torch.float32, rows=4096):
    """torch_reference's mean loss and gradients (eps = z = 0, no bias) with
    the logits materialised `rows` rows at a time: autograd runs per row
    chunk, the weight gradient accumulates across chunks and every chunk's
    objective is divided by the global labelled-row count.  This keeps a
    full-size reference within a few GB of device memory.
    """
    d = hidden.shape[-1]
    h = hidden.detach().reshape(-1, d)
    lab = labels.reshape(-1)
    N, V = h.shape[0], weight.shape[0]
    w = weight.detach().to(dtype).requires_grad_(True)
    n_valid = max(int((lab != ignore_index).sum().item()), 1)
    dh = torch.empty(N, d, dtype=dtype, device=h.device)
    loss = torch.zeros((), dtype=torch.float64, device=h.device)
    for r0 in range(0, N, rows):
        hc = h[r0:r0 + rows].to(dtype).requires_grad_(True)
        lc = lab[r0:r0 + rows]
        logits = hc @ w.t()
        valid = lc != ignore_index
        in_range = valid & (lc >= 0) & (lc < V)
        lse = torch.logsumexp(logits, dim=-1)
        tgt = logits.gather(1, torch.where(in_range, lc, torch.zeros_like(lc))[:, None])[:, 0] * in_range.to(dtype)
        obj = ((lse - tgt) * valid.to(dtype)).sum() / n_valid
        obj.backward()
        dh[r0:r0 + rows] = hc.grad
        loss += obj.detach().double()
        del logits, lse, tgt, obj, hc
    return {"loss": loss, "dh": dh.reshape(hidden.shape), "dw": w.grad.detach()}


def grad_report_torch(got: torch.Tensor, ref: torch.Tensor) -> dict:
    """grad_report computed on the tensors' device in float64."""
    g = got.detach().reshape(-1).double()
    r = ref.detach().reshape(-1).to(g.device).double()
    scale = float(r.abs().max()) if r.numel() else 0.0
    err = float((g - r).abs().max()) if r.numel() else 0.0
    ng, nr = float(g.norm()), float(r.norm())
    cos = 1.0 if ng == 0 and nr == 0 else (0.0 if ng == 0 or nr == 0 else float(g @ r) / (ng * nr))
    return {"max_abs_err": err, "max_ref": scale, "frac": err / scale if scale > 0 else err, "cos": cos}


def assert_grad_close_torch(got: torch.Tensor, ref: torch.Tensor, what: str):
    r = grad_report_torch(got, ref)
    if r["max_ref"] == 0.0:
        assert r["max_abs_err"] <= 1e-6, f"{what}: expected zeros, {r}"
        return
    assert r["frac"] <= GRAD_MAXABS_FRAC, f"{what}: max abs err too large {r}"
    assert r["cos"] >= GRAD_COS_MIN, f"{what}: cosine too small {r}"

