"""CPU oracle for the Cut Cross-Entropy path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker.  The product path
(chronicals_amd) never calls it.

A numpy restatement of the reference's PyTorch CPU algorithm
(Ajwebdevs/Chronicals v0.1.4, chronicals/kernels/cut_cross_entropy.py):

  forward()   follows CutCrossEntropyForward.forward, :567-692
              V-chunked logits (:627-637), online max / rescaled sum-exp with
              Kahan compensation (:641-660), target gather (:663-668),
              lse = m + log(s + 1e-10) (:671), ce = lse - t (:674),
              label smoothing (1-eps)*ce + eps*log(V) (:677-679),
              z-loss z*lse^2 (:682-683), mask (:686), reductions
              mean = sum/max(n_valid,1) (:688-690) and 'sum'/'none' as in
              triton_kernels.py:2481-2491.  smoothing='uniform' gives the
              loss of triton_fused_linear_cross_entropy
              (triton_kernels.py:3147-3263, whose rows go through
              _liger_ce_kernel :2914-2956): eps*(lse - mean_v logits)
              in place of eps*log(V); its gradient is backward()'s.
  backward()  follows CutCrossEntropyBackward.backward, :703-808
              recompute logits per chunk (:762), P = exp(S - lse) (:767),
              G = P - (1-eps)*onehot (:773-780) - eps/V (:783-784)
              + 2z*lse*P (:787-789), times valid * grad_out/n_valid (:745,
              :792); dH += G W_c (:795), dW_c = G^T H (:798), dB_c = sum G
              (:801-802).

  logits_forward()   cross-entropy over existing logits [N, V]:
              smoothing='logv' follows chunked_cross_entropy_loss,
              cut_cross_entropy.py:1199-1249: per V-chunk online max and
              rescaled sum-exp (:1210-1221), lse = m + log(s + 1e-10) (:1223),
              target gather with ignored rows zeroed (:1226-1231),
              (1-eps)*ce + eps*log(V) (:1234-1239), z*lse^2 (:1242-1243),
              mask and sum / max(n_valid, 1) (:1246-1249).
              smoothing='uniform' follows _liger_ce_kernel,
              triton_kernels.py:2886-2963: the same online pass per block
              (:2893-2911) plus smooth_sum = -eps/V * sum(x) (:2914-2915),
              loss = (1-eps)*(lse - t) + smooth_sum + eps*lse (:2952-2956),
              + z*lse^2 (:2959); which is also fused_cross_entropy_kernel's
              loss (:175-194).
  logits_backward()  dLoss/dlogits of logits_forward(): 'logv' is what
              autograd gives through :1199-1249, (1-eps)*(p - onehot)
              + 2z*lse*p; 'uniform' is :2930-2947 (and :197-206),
              p - eps/V - (1-eps)*onehot + 2z*lse*p; times g_n
              (grad_out, divided by max(n_valid, 1) for 'mean', :2946-2947).

The reference's CPU backward loses the one-hot term: its scatter_add_ at
:776-780 writes into a boolean-mask copy.  backward() applies the term by
default (as the reference's GPU path, :530-546, and its sibling
FusedLinearCrossEntropyFunction, triton_kernels.py:2594-2601, do);
``apply_onehot=False`` reproduces the as-shipped CPU gradient and exists only
so tests can show the pinning checks reject it.

Parity pins (tests/test_oracle.py, tests/test_oracle_logits.py): every
function here is checked against
an independent float64 closed form (torch's logsumexp / cross_entropy with
autograd, including torch's own label_smoothing, and brute-force Python sums
on tiny inputs), special cases (W = 0 gives loss log V; all rows ignored
gives 0) and invariants (sum over the vocabulary of G is 0 when eps = z = 0).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

REDUCTIONS = ("mean", "sum", "none")


def _flat(hidden: np.ndarray, labels: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    d = hidden.shape[-1]
    return hidden.reshape(-1, d), labels.reshape(-1)


def forward(hidden: np.ndarray, weight: np.ndarray, labels: np.ndarray, bias: Optional[np.ndarray] = None,
            chunk_size: int = 8192, ignore_index: int = -100, label_smoothing: float = 0.0,
            z_loss_weight: float = 0.0, use_kahan: bool = True, reduction: str = "mean",
            dtype=np.float32, smoothing: str = "logv"):
    """Returns (loss, lse [N], target_logit [N], valid_mask [N])."""
    if reduction not in REDUCTIONS:
        raise ValueError(reduction)
    if smoothing not in ("logv", "uniform"):
        raise ValueError(smoothing)
    h, lab = _flat(np.asarray(hidden), np.asarray(labels))
    h = h.astype(dtype, copy=False)
    w = np.asarray(weight).astype(dtype, copy=False)
    b = None if bias is None else np.asarray(bias).astype(dtype, copy=False)
    n = h.shape[0]
    V = w.shape[0]
    max_logit = np.full(n, -np.inf, dtype=dtype)
    sum_exp = np.zeros(n, dtype=dtype)
    comp = np.zeros(n, dtype=dtype)
    target = np.zeros(n, dtype=dtype)
    row_sum = np.zeros(n, dtype=np.float64)
    valid = lab != ignore_index
    for c0 in range(0, V, chunk_size):
        c1 = min(c0 + chunk_size, V)
        logits = h @ w[c0:c1].T
        if b is not None:
            logits = logits + b[c0:c1]
        if smoothing == "uniform":
            row_sum += logits.sum(axis=1, dtype=np.float64)
        cmax = logits.max(axis=1) if n else np.zeros(0, dtype)
        new_max = np.maximum(max_logit, cmax)
        sum_exp = sum_exp * np.exp(max_logit - new_max)
        csum = np.exp(logits - new_max[:, None]).sum(axis=1, dtype=dtype)
        if use_kahan:
            y = csum - comp
            t = sum_exp + y
            comp = (t - sum_exp) - y
            sum_exp = t
        else:
            sum_exp = sum_exp + csum
        max_logit = new_max
        in_chunk = valid & (lab >= c0) & (lab < c1)
        if in_chunk.any():
            rows = np.nonzero(in_chunk)[0]
            target[rows] = logits[rows, lab[rows] - c0]
    lse = (max_logit + np.log(sum_exp + dtype(1e-10))).astype(dtype)
    ce = lse - target
    if label_smoothing > 0.0:
        smooth = math.log(V) if smoothing == "logv" else (lse - row_sum / V).astype(dtype)
        ce = (1.0 - label_smoothing) * ce + label_smoothing * smooth
    total = (ce + z_loss_weight * lse ** 2).astype(dtype)
    total = total * valid.astype(dtype)
    n_valid = max(int(valid.sum()), 1)
    if reduction == "mean":
        loss = dtype(total.sum(dtype=np.float64) / n_valid)
    elif reduction == "sum":
        loss = dtype(total.sum(dtype=np.float64))
    else:
        loss = total
    return loss, lse, target, valid


def backward(hidden: np.ndarray, weight: np.ndarray, labels: np.ndarray, lse: np.ndarray, valid_mask: np.ndarray,
             grad_output, bias: Optional[np.ndarray] = None, chunk_size: int = 8192, ignore_index: int = -100,
             label_smoothing: float = 0.0, z_loss_weight: float = 0.0, reduction: str = "mean",
             apply_onehot: bool = True, dtype=np.float32):
    """Returns (grad_hidden [N,d], grad_weight [V,d], grad_bias [V] or None)."""
    del ignore_index  # valid_mask carries it
    h, lab = _flat(np.asarray(hidden), np.asarray(labels))
    h = h.astype(dtype, copy=False)
    w = np.asarray(weight).astype(dtype, copy=False)
    b = None if bias is None else np.asarray(bias).astype(dtype, copy=False)
    n, d = h.shape
    V = w.shape[0]
    valid = np.asarray(valid_mask).reshape(-1)
    lse = np.asarray(lse, dtype=dtype).reshape(-1)
    go = np.asarray(grad_output, dtype=np.float64).reshape(-1)
    n_valid = max(int(valid.sum()), 1)
    if reduction == "mean":
        scale = np.full(n, go[0] / n_valid)
    elif reduction == "sum":
        scale = np.full(n, go[0])
    else:
        scale = go.copy()
    scale = (scale * valid).astype(dtype)
    gh = np.zeros((n, d), dtype=dtype)
    gw = np.zeros((V, d), dtype=dtype)
    gb = np.zeros(V, dtype=dtype) if b is not None else None
    for c0 in range(0, V, chunk_size):
        c1 = min(c0 + chunk_size, V)
        wc = w[c0:c1]
        logits = h @ wc.T
        if b is not None:
            logits = logits + b[c0:c1]
        probs = np.exp(logits - lse[:, None])
        g = probs.copy()
        if apply_onehot:
            in_chunk = valid & (lab >= c0) & (lab < c1)
            rows = np.nonzero(in_chunk)[0]
            g[rows, lab[rows] - c0] -= dtype(1.0 - label_smoothing)
        if label_smoothing > 0.0:
            g = g - dtype(label_smoothing / V)
        if z_loss_weight > 0.0:
            g = g + dtype(2.0 * z_loss_weight) * lse[:, None] * probs
        g = (g * scale[:, None]).astype(dtype)
        gh += g @ wc
        gw[c0:c1] = g.T @ h
        if gb is not None:
            gb[c0:c1] = g.sum(axis=0)
    return gh, gw, gb


def loss_and_grads(hidden, weight, labels, bias=None, chunk_size=8192, ignore_index=-100, label_smoothing=0.0,
                   z_loss_weight=0.0, reduction="mean", grad_output=None, dtype=np.float32, smoothing="logv"):
    """forward() then backward() with grad_output (default 1 / ones)."""
    loss, lse, _, valid = forward(hidden, weight, labels, bias, chunk_size, ignore_index, label_smoothing,
                                  z_loss_weight, True, reduction, dtype, smoothing)
    if grad_output is None:
        grad_output = np.ones(np.asarray(labels).size) if reduction == "none" else np.ones(1)
    gh, gw, gb = backward(hidden, weight, labels, lse, valid, grad_output, bias, chunk_size, ignore_index,
                          label_smoothing, z_loss_weight, reduction, True, dtype)
    return loss, lse, gh, gw, gb


SMOOTHING_FORMS = ("logv", "uniform")


def logits_forward(logits: np.ndarray, labels: np.ndarray, chunk_size: int = 8192, ignore_index: int = -100,
                   label_smoothing: float = 0.0, z_loss_weight: float = 0.0, reduction: str = "mean",
                   smoothing: str = "logv", dtype=np.float32):
    """Cross-entropy over logits [..., V].  Returns (loss, lse [N], valid_mask [N])."""
    if reduction not in REDUCTIONS:
        raise ValueError(reduction)
    if smoothing not in SMOOTHING_FORMS:
        raise ValueError(smoothing)
    x = np.asarray(logits)
    V = x.shape[-1]
    x = x.reshape(-1, V).astype(dtype, copy=False)
    lab = np.asarray(labels).reshape(-1)
    n = x.shape[0]
    max_logit = np.full(n, -np.inf, dtype=dtype)
    sum_exp = np.zeros(n, dtype=dtype)
    smooth_sum = np.zeros(n, dtype=dtype)
    for c0 in range(0, V, chunk_size):
        xc = x[:, c0:min(c0 + chunk_size, V)]
        cmax = xc.max(axis=1) if n else np.zeros(0, dtype)
        new_max = np.maximum(max_logit, cmax)
        sum_exp = sum_exp * np.exp(max_logit - new_max)
        max_logit = new_max
        sum_exp = sum_exp + np.exp(xc - max_logit[:, None]).sum(axis=1, dtype=dtype)
        if smoothing == "uniform":
            smooth_sum = smooth_sum + (dtype(-label_smoothing / V) * xc).sum(axis=1, dtype=dtype)
    lse = (max_logit + np.log(sum_exp + dtype(1e-10))).astype(dtype)
    valid = lab != ignore_index
    has_t = valid & (lab >= 0) & (lab < V)
    target = np.zeros(n, dtype=dtype)
    rows = np.nonzero(has_t)[0]
    target[rows] = x[rows, lab[rows]]
    ce = lse - target
    if smoothing == "logv":
        if label_smoothing > 0.0:
            ce = (1.0 - label_smoothing) * ce + label_smoothing * math.log(V)
    elif label_smoothing > 0.0:
        ce = ce * (1.0 - label_smoothing) + (smooth_sum + label_smoothing * lse)
    total = (ce + z_loss_weight * lse ** 2).astype(dtype) * valid.astype(dtype)
    n_valid = max(int(valid.sum()), 1)
    if reduction == "mean":
        loss = dtype(total.sum(dtype=np.float64) / n_valid)
    elif reduction == "sum":
        loss = dtype(total.sum(dtype=np.float64))
    else:
        loss = total
    return loss, lse, valid


def logits_backward(logits: np.ndarray, labels: np.ndarray, lse: np.ndarray, valid_mask: np.ndarray, grad_output,
                    label_smoothing: float = 0.0, z_loss_weight: float = 0.0, reduction: str = "mean",
                    smoothing: str = "logv", dtype=np.float32) -> np.ndarray:
    """dLoss/dlogits [N, V] of logits_forward() times grad_output."""
    if smoothing not in SMOOTHING_FORMS:
        raise ValueError(smoothing)
    x = np.asarray(logits)
    V = x.shape[-1]
    x = x.reshape(-1, V).astype(dtype, copy=False)
    lab = np.asarray(labels).reshape(-1)
    n = x.shape[0]
    valid = np.asarray(valid_mask).reshape(-1)
    lse = np.asarray(lse, dtype=dtype).reshape(-1)
    go = np.asarray(grad_output, dtype=np.float64).reshape(-1)
    n_valid = max(int(valid.sum()), 1)
    if reduction == "mean":
        scale = np.full(n, go[0] / n_valid)
    elif reduction == "sum":
        scale = np.full(n, go[0])
    else:
        scale = go.copy()
    scale = (scale * valid).astype(dtype)
    p = np.exp(x - lse[:, None])
    eps = label_smoothing
    if smoothing == "logv":
        g = dtype(1.0 - eps) * p
    else:
        g = p - dtype(eps / V)
    if z_loss_weight > 0.0:
        g = g + dtype(2.0 * z_loss_weight) * lse[:, None] * p
    rows = np.nonzero(valid & (lab >= 0) & (lab < V))[0]
    g[rows, lab[rows]] -= dtype(1.0 - eps)
    return (g * scale[:, None]).astype(dtype)
