"""Pins the logits-in oracle (oracle.cce_oracle.logits_forward / logits_backward).

Checks that do not restate the oracle:
* torch's own cross_entropy (float64), with its label_smoothing, for the
  uniform-target form and for eps = 0 in both forms;
* float64 autograd of the reference's expressions (cut_cross_entropy.py:
  1199-1249 for 'logv'; triton_kernels.py:2952-2959 for 'uniform'), written
  with torch.logsumexp rather than the oracle's online chunked pass;
* brute-force Python sums on tiny inputs;
* special cases (constant logits give loss log V in both forms and for any
  eps; all rows ignored gives 0) and invariants (each row's gradient sums to 0
  when z = 0; ignored rows have zero gradient);
* planted mistakes (the other smoothing form's gradient, a flipped one-hot
  sign, a dropped z term) that the checks must reject.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cce_oracle as oracle
from tests.cce_common import IGNORE


def _case(N=41, V=503, seed=0, ignore_frac=0.2, oob=False, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, V, generator=g) * scale
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < ignore_frac] = IGNORE
    if oob:
        lab[1] = V + 3
        lab[2] = -5
    return x, lab


def torch_closed_form(x, lab, eps=0.0, z=0.0, reduction="mean", smoothing="logv", grad_output=None):
    """float64 loss and autograd gradient of the reference expression."""
    x = x.detach().double().requires_grad_(True)
    V = x.shape[-1]
    valid = lab != IGNORE
    has_t = valid & (lab >= 0) & (lab < V)
    lse = torch.logsumexp(x, dim=-1)
    t = x.gather(1, torch.where(has_t, lab, 0)[:, None])[:, 0] * has_t.double()
    if smoothing == "logv":
        row = (1 - eps) * (lse - t) + eps * math.log(V)
    else:
        row = (1 - eps) * (lse - t) + eps * (lse - x.mean(dim=-1))
    row = (row + z * lse * lse) * valid.double()
    nv = max(int(valid.sum()), 1)
    if reduction == "mean":
        loss = row.sum() / nv
    elif reduction == "sum":
        loss = row.sum()
    else:
        loss = row
    go = torch.ones_like(loss) if grad_output is None else torch.as_tensor(grad_output, dtype=torch.float64)
    (gx,) = torch.autograd.grad(loss, x, go.reshape(loss.shape))
    return loss.detach().numpy(), lse.detach().numpy(), gx.numpy()


def run_oracle(x, lab, eps=0.0, z=0.0, reduction="mean", smoothing="logv", chunk=8192, grad_output=None,
               dtype=np.float64):
    loss, lse, valid = oracle.logits_forward(x.numpy(), lab.numpy(), chunk, IGNORE, eps, z, reduction, smoothing,
                                             dtype)
    if grad_output is None:
        grad_output = np.ones(lab.numel()) if reduction == "none" else np.ones(1)
    g = oracle.logits_backward(x.numpy(), lab.numpy(), lse, valid, grad_output, eps, z, reduction, smoothing, dtype)
    return loss, lse, g


@pytest.mark.parametrize("smoothing", ["logv", "uniform"])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("eps,z", [(0.0, 0.0), (0.1, 0.0), (0.0, 1e-3), (0.2, 1e-2)])
@pytest.mark.parametrize("chunk", [64, 8192])
def test_logits_oracle_matches_float64_autograd(smoothing, reduction, eps, z, chunk):
    x, lab = _case(oob=True)
    go = None if reduction != "none" else torch.rand(x.shape[0], generator=torch.Generator().manual_seed(5)).numpy()
    rl, rlse, rg = torch_closed_form(x, lab, eps, z, reduction, smoothing, go)
    loss, lse, g = run_oracle(x, lab, eps, z, reduction, smoothing, chunk, go)
    # the oracle's lse carries the reference's + 1e-10 inside the log (sum >= 1, so <= 1e-10 relative)
    np.testing.assert_allclose(loss, rl, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(lse, rlse, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(g, rg, rtol=1e-8, atol=1e-14)


@pytest.mark.parametrize("eps", [0.0, 0.1, 0.3])
def test_uniform_form_is_torch_label_smoothed_cross_entropy(eps):
    # torch's own label smoothing is the uniform-target form (triton_kernels.py:189-193)
    x, lab = _case(N=64, V=777, seed=1)
    xd = x.double().requires_grad_(True)
    ref = F.cross_entropy(xd, lab, ignore_index=IGNORE, label_smoothing=eps)
    (rg,) = torch.autograd.grad(ref, xd)
    loss, _, g = run_oracle(x, lab, eps, 0.0, "mean", "uniform")
    np.testing.assert_allclose(loss, ref.item(), rtol=1e-9)
    np.testing.assert_allclose(g, rg.numpy(), rtol=1e-8, atol=1e-15)


def test_logv_form_without_smoothing_is_torch_cross_entropy():
    x, lab = _case(N=64, V=777, seed=2)
    xd = x.double().requires_grad_(True)
    ref = F.cross_entropy(xd, lab, ignore_index=IGNORE)
    (rg,) = torch.autograd.grad(ref, xd)
    loss, _, g = run_oracle(x, lab, 0.0, 0.0, "mean", "logv")
    np.testing.assert_allclose(loss, ref.item(), rtol=1e-9)
    np.testing.assert_allclose(g, rg.numpy(), rtol=1e-8, atol=1e-15)


@pytest.mark.parametrize("smoothing", ["logv", "uniform"])
def test_logits_oracle_brute_force_tiny(smoothing):
    x, lab = _case(N=5, V=7, seed=3, ignore_frac=0.3)
    eps, z = 0.15, 0.05
    xs, ls = x.double().tolist(), lab.tolist()
    rows, grads = [], []
    for r, t in zip(xs, ls):
        if t == IGNORE:
            rows.append(0.0)
            grads.append([0.0] * len(r))
            continue
        lse = math.log(sum(math.exp(v) for v in r))
        smooth = math.log(len(r)) if smoothing == "logv" else lse - sum(r) / len(r)
        rows.append((1 - eps) * (lse - r[t]) + eps * smooth + z * lse * lse)
        gr = []
        for j, v in enumerate(r):
            p = math.exp(v - lse)
            if smoothing == "logv":
                gj = (1 - eps) * p + 2 * z * lse * p
            else:
                gj = p - eps / len(r) + 2 * z * lse * p
            if j == t:
                gj -= 1 - eps
            gr.append(gj)
        grads.append(gr)
    nv = max(sum(1 for t in ls if t != IGNORE), 1)
    loss, _, g = run_oracle(x, lab, eps, z, "mean", smoothing)
    assert abs(float(loss) - sum(rows) / nv) < 1e-9
    np.testing.assert_allclose(g, np.array(grads) / nv, rtol=1e-8, atol=1e-15)


@pytest.mark.parametrize("smoothing", ["logv", "uniform"])
@pytest.mark.parametrize("eps", [0.0, 0.25])
def test_constant_logits_give_log_vocab(smoothing, eps):
    V = 1000
    x = torch.full((6, V), 3.5)
    lab = torch.tensor([0, 5, 999, IGNORE, 17, 400])
    loss, lse, _ = run_oracle(x, lab, eps, 0.0, "mean", smoothing)
    np.testing.assert_allclose(lse, 3.5 + math.log(V), rtol=1e-9)
    np.testing.assert_allclose(loss, math.log(V), rtol=1e-9)


@pytest.mark.parametrize("smoothing", ["logv", "uniform"])
def test_logits_oracle_all_ignored(smoothing):
    x, _ = _case(N=9, V=50)
    lab = torch.full((9,), IGNORE)
    loss, _, g = run_oracle(x, lab, 0.1, 0.01, "mean", smoothing)
    assert loss == 0.0
    assert not g.any()


@pytest.mark.parametrize("smoothing", ["logv", "uniform"])
def test_logits_gradient_rows_sum_to_zero(smoothing):
    x, lab = _case(oob=False)
    _, _, g = run_oracle(x, lab, 0.2, 0.0, "sum", smoothing)
    # softmax sums to s / (s + 1e-10) with the reference's 1e-10 inside the log
    np.testing.assert_allclose(g.sum(axis=1), 0.0, atol=1e-9)
    assert not g[(lab == IGNORE).numpy()].any()


def test_logits_out_of_range_labels_have_no_target():
    x, lab = _case(N=6, V=40, seed=4, ignore_frac=0.0, oob=True)
    loss, lse, g = run_oracle(x, lab, 0.0, 0.0, "none", "logv")
    np.testing.assert_allclose(loss[1:3], lse[1:3], rtol=1e-9)
    p = np.exp(x.double().numpy() - lse[:, None])
    np.testing.assert_allclose(g[1:3], p[1:3], rtol=1e-10)


def test_logits_oracle_fp32_close_to_fp64():
    x, lab = _case(N=33, V=4097, seed=6)
    l32, lse32, g32 = run_oracle(x, lab, 0.1, 1e-3, "mean", "uniform", dtype=np.float32)
    l64, lse64, g64 = run_oracle(x, lab, 0.1, 1e-3, "mean", "uniform", dtype=np.float64)
    np.testing.assert_allclose(l32, l64, rtol=1e-5)
    np.testing.assert_allclose(lse32, lse64, rtol=1e-6)
    np.testing.assert_allclose(g32, g64, rtol=1e-4, atol=1e-9)


def test_planted_mistakes_are_rejected():
    x, lab = _case(seed=7)
    eps, z = 0.2, 0.05
    _, _, ref_logv = torch_closed_form(x, lab, eps, z, "mean", "logv")
    _, _, ref_uni = torch_closed_form(x, lab, eps, z, "mean", "uniform")
    # the other form's gradient
    _, _, g_uni = run_oracle(x, lab, eps, z, "mean", "uniform")
    _, _, g_logv = run_oracle(x, lab, eps, z, "mean", "logv")
    assert not np.allclose(g_uni, ref_logv, rtol=1e-6, atol=1e-9)
    assert not np.allclose(g_logv, ref_uni, rtol=1e-6, atol=1e-9)
    # a flipped one-hot sign
    valid = (lab != IGNORE).numpy()
    rows = np.nonzero(valid)[0]
    flipped = g_logv.copy()
    flipped[rows, lab.numpy()[rows]] += 2 * (1 - eps) / valid.sum()
    assert not np.allclose(flipped, ref_logv, rtol=1e-6, atol=1e-9)
    # a dropped z term
    _, _, g_noz = run_oracle(x, lab, eps, 0.0, "mean", "logv")
    assert not np.allclose(g_noz, ref_logv, rtol=1e-6, atol=1e-9)
    # and the loss forms differ too
    l_uni, _, _ = run_oracle(x, lab, eps, z, "mean", "uniform")
    l_ref, _, _ = torch_closed_form(x, lab, eps, z, "mean", "logv")
    assert abs(float(l_uni) - float(l_ref)) > 1e-6
