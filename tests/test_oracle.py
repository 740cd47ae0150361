"""Pins the CPU oracle (oracle/cce_oracle.py) to checks that do not restate it.

* float64 closed forms built from torch's logsumexp / cross_entropy and
  autograd (an independent library implementation);
* brute-force Python sums on tiny inputs;
* special cases with textbook answers (W = 0 -> loss = log V; all rows
  ignored -> loss 0 and zero gradients);
* invariants (sum over the vocabulary of dLoss/dlogits is 0 when eps = z = 0,
  so sum_v dW[v] = 0 and sum_v dB[v] = 0);
* a planted mistake (the reference CPU backward's lost one-hot term) that the
  checks must reject.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cce_oracle as oracle
from tests.cce_common import IGNORE, torch_reference


def _case(N=37, d=24, V=1000, seed=0, ignore_frac=0.2, bias=False, oob=False):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(N, d, generator=g)
    w = torch.randn(V, d, generator=g) * 0.3
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < ignore_frac] = IGNORE
    if oob:
        lab[1] = V + 5
        lab[2] = -7
    b = torch.randn(V, generator=g) * 0.5 if bias else None
    return h, w, lab, b


def _np(t):
    return None if t is None else t.detach().cpu().numpy()


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("chunk", [64, 333, 8192])
def test_oracle_matches_float64_closed_form(reduction, bias, chunk):
    h, w, lab, b = _case(bias=bias)
    ref = torch_reference(h, w, lab, b, reduction=reduction)
    loss, lse, gh, gw, gb = oracle.loss_and_grads(_np(h), _np(w), _np(lab), _np(b), chunk_size=chunk,
                                                  reduction=reduction)
    np.testing.assert_allclose(loss, ref["loss"].numpy(), rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(lse, ref["lse"].numpy(), rtol=2e-6, atol=2e-5)
    np.testing.assert_allclose(gh, ref["dh"].numpy(), rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(gw, ref["dw"].numpy(), rtol=1e-4, atol=2e-6)
    if bias:
        np.testing.assert_allclose(gb, ref["db"].numpy(), rtol=1e-4, atol=2e-6)


def test_oracle_mean_equals_torch_cross_entropy():
    # The exact comparison the reference's own self-test makes (cut_cross_entropy.py:1487-1490).
    h, w, lab, _ = _case(N=64, d=32, V=777)
    ce = F.cross_entropy((h.double() @ w.double().t()), lab, ignore_index=IGNORE)
    loss, *_ = oracle.forward(_np(h), _np(w), _np(lab), chunk_size=100)
    assert abs(float(loss) - ce.item()) < 1e-5


@pytest.mark.parametrize("eps,z", [(0.1, 0.0), (0.0, 1e-2), (0.2, 1e-3)])
def test_oracle_smoothing_and_zloss(eps, z):
    h, w, lab, b = _case(N=29, d=16, V=501, seed=3, bias=True)
    ref = torch_reference(h, w, lab, b, label_smoothing=eps, z_loss_weight=z)
    loss, lse, gh, gw, gb = oracle.loss_and_grads(_np(h), _np(w), _np(lab), _np(b), chunk_size=128,
                                                  label_smoothing=eps, z_loss_weight=z)
    np.testing.assert_allclose(loss, ref["loss"].numpy(), rtol=2e-5)
    np.testing.assert_allclose(gh, ref["dh"].numpy(), rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(gw, ref["dw"].numpy(), rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(gb, ref["db"].numpy(), rtol=1e-4, atol=2e-6)


def test_torch_label_smoothing_gradient_is_reference_gradient():
    """The smoothed-loss gradient P - (1-eps)onehot - eps/V equals torch's label_smoothing CE gradient."""
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(6, 11, generator=g, dtype=torch.float64, requires_grad=True)
    lab = torch.randint(0, 11, (6,), generator=g)
    eps = 0.3
    F.cross_entropy(logits, lab, label_smoothing=eps, reduction="sum").backward()
    p = torch.softmax(logits.detach(), -1)
    expect = p - (1 - eps) * F.one_hot(lab, 11).double() - eps / 11
    torch.testing.assert_close(logits.grad, expect)


def test_oracle_brute_force_tiny():
    rng = np.random.default_rng(7)
    N, d, V = 3, 4, 7
    h = rng.standard_normal((N, d)).astype(np.float32)
    w = rng.standard_normal((V, d)).astype(np.float32)
    lab = np.array([2, IGNORE, 6])
    eps, z = 0.25, 0.05
    S = [[math.fsum(float(h[n, k]) * float(w[v, k]) for k in range(d)) for v in range(V)] for n in range(N)]
    lse = [math.log(math.fsum(math.exp(s) for s in row)) for row in S]
    rows = []
    for n in range(N):
        if lab[n] == IGNORE:
            continue
        ce = lse[n] - S[n][lab[n]]
        rows.append((1 - eps) * ce + eps * math.log(V) + z * lse[n] ** 2)
    expect_loss = math.fsum(rows) / len(rows)
    # dlogits by central finite differences of the smoothed objective with (lse - mean S)
    def obj(Sm):
        tot = 0.0
        for n in range(N):
            if lab[n] == IGNORE:
                continue
            l_ = math.log(math.fsum(math.exp(s) for s in Sm[n]))
            tot += (1 - eps) * (l_ - Sm[n][lab[n]]) + eps * (l_ - math.fsum(Sm[n]) / V) + z * l_ ** 2
        return tot / len(rows)
    G = np.zeros((N, V))
    for n in range(N):
        for v in range(V):
            Sp = [r[:] for r in S]
            Sn = [r[:] for r in S]
            Sp[n][v] += 1e-6
            Sn[n][v] -= 1e-6
            G[n, v] = (obj(Sp) - obj(Sn)) / 2e-6
    loss, lse_o, gh, gw, _ = oracle.loss_and_grads(h, w, lab, chunk_size=3, label_smoothing=eps, z_loss_weight=z,
                                                   dtype=np.float64)
    assert abs(loss - expect_loss) < 1e-10
    # the reference's lse is m + log(s + 1e-10) (:671): an offset of at most 1e-10/s
    np.testing.assert_allclose(lse_o, lse, rtol=0, atol=1e-10)
    np.testing.assert_allclose(gh, G @ w.astype(np.float64), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(gw, G.T @ h.astype(np.float64), rtol=1e-6, atol=1e-8)


def test_oracle_zero_weight_gives_log_vocab():
    h, _, lab, _ = _case(N=16, d=8, V=321)
    w = np.zeros((321, 8), np.float32)
    loss, lse, gh, gw, _ = oracle.loss_and_grads(_np(h), w, _np(lab), chunk_size=100)
    assert abs(float(loss) - math.log(321)) < 1e-5
    np.testing.assert_allclose(lse, math.log(321), rtol=1e-6)
    np.testing.assert_array_equal(gh, 0.0)
    # G = 1/V - onehot per valid row, so dW = G^T H
    lab_np = _np(lab)
    valid = lab_np != IGNORE
    G = np.zeros((16, 321))
    G[valid] = 1.0 / 321
    G[np.nonzero(valid)[0], lab_np[valid]] -= 1.0
    G /= valid.sum()
    np.testing.assert_allclose(gw, G.T @ _np(h), rtol=1e-4, atol=1e-7)


def test_oracle_all_ignored():
    h, w, lab, b = _case(N=8, d=8, V=50, bias=True)
    lab[:] = IGNORE
    for red in ("mean", "sum"):
        loss, lse, gh, gw, gb = oracle.loss_and_grads(_np(h), _np(w), _np(lab), _np(b), reduction=red)
        assert float(loss) == 0.0
        assert not gh.any() and not gw.any() and not gb.any()


def test_oracle_out_of_range_labels_have_no_target():
    h, w, lab, _ = _case(N=10, d=8, V=40, ignore_frac=0.0, oob=True)
    loss, lse, target, valid = oracle.forward(_np(h), _np(w), _np(lab), chunk_size=16, reduction="none")
    assert valid[1] and valid[2]
    assert target[1] == 0.0 and target[2] == 0.0
    np.testing.assert_allclose(loss[1:3], lse[1:3], rtol=1e-6)
    ref = torch_reference(h, w, lab, reduction="none")
    np.testing.assert_allclose(loss, ref["loss"].numpy(), rtol=1e-5, atol=1e-6)
    _, _, gh, gw, _ = oracle.loss_and_grads(_np(h), _np(w), _np(lab), chunk_size=16, reduction="mean")
    ref = torch_reference(h, w, lab, reduction="mean")
    np.testing.assert_allclose(gh, ref["dh"].numpy(), rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(gw, ref["dw"].numpy(), rtol=1e-4, atol=1e-6)


def test_oracle_gradient_sums_to_zero_over_vocab():
    h, w, lab, b = _case(N=33, d=12, V=257, bias=True)
    _, _, gh, gw, gb = oracle.loss_and_grads(_np(h), _np(w), _np(lab), _np(b), chunk_size=50)
    assert abs(gb.sum()) < 1e-6
    np.testing.assert_allclose(gw.sum(axis=0), 0.0, atol=1e-6)


def test_oracle_chunk_size_independent():
    h, w, lab, b = _case(N=20, d=16, V=999, bias=True)
    a = oracle.loss_and_grads(_np(h), _np(w), _np(lab), _np(b), chunk_size=37)
    c = oracle.loss_and_grads(_np(h), _np(w), _np(lab), _np(b), chunk_size=100000)
    for x, y in zip(a, c):
        np.testing.assert_allclose(x, y, rtol=2e-5, atol=1e-7)


def test_planted_reference_bug_is_rejected():
    """The as-shipped CPU backward (no one-hot term) must fail the closed-form check."""
    h, w, lab, _ = _case()
    ref = torch_reference(h, w, lab)
    loss, lse, _, valid = oracle.forward(_np(h), _np(w), _np(lab))
    gh, gw, _ = oracle.backward(_np(h), _np(w), _np(lab), lse, valid, np.ones(1), apply_onehot=False)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(gh, ref["dh"].numpy(), rtol=1e-3, atol=1e-5)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(gw, ref["dw"].numpy(), rtol=1e-3, atol=1e-5)


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_oracle_uniform_smoothing_is_torch_label_smoothed_cross_entropy(bias, reduction):
    # the loss of triton_fused_linear_cross_entropy (_liger_ce_kernel, triton_kernels.py:2914-2956) is torch's
    # label-smoothed cross-entropy of the logits plus z*lse^2; the oracle forms the row mean of the logits per chunk
    h, w, lab, b = _case(N=33, d=24, V=777, seed=8, bias=bias)
    eps, z = 0.2, 1e-3
    logits = h.double() @ w.double().t() + (b.double() if bias else 0.0)
    rows = F.cross_entropy(logits, lab, ignore_index=IGNORE, label_smoothing=eps, reduction="none")
    rows = (rows + z * torch.logsumexp(logits, -1) ** 2) * (lab != IGNORE).double()
    nv = max(int((lab != IGNORE).sum()), 1)
    ref = {"mean": rows.sum() / nv, "sum": rows.sum(), "none": rows}[reduction].numpy()
    for chunk in (100, 8192):
        loss, *_ = oracle.forward(_np(h), _np(w), _np(lab), _np(b), chunk_size=chunk, label_smoothing=eps,
                                  z_loss_weight=z, reduction=reduction, dtype=np.float64, smoothing="uniform")
        np.testing.assert_allclose(loss, ref, rtol=1e-9, atol=1e-12)
    # the eps*log(V) form differs from it whenever eps > 0 (the check tells the two apart)
    lv, *_ = oracle.forward(_np(h), _np(w), _np(lab), _np(b), label_smoothing=eps, z_loss_weight=z,
                            reduction="sum", dtype=np.float64)
    assert abs(float(lv) - float(rows.sum())) > 1e-3


def test_oracle_uniform_smoothing_gradient_is_its_autograd():
    # backward()'s P - (1-eps)onehot - eps/V + 2z*lse*P is the exact derivative of the uniform-form loss
    h, w, lab, b = _case(N=21, d=16, V=301, seed=9, bias=True)
    eps, z = 0.15, 1e-2
    hd = h.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    bd = b.double().requires_grad_(True)
    logits = hd @ wd.t() + bd
    rows = F.cross_entropy(logits, lab, ignore_index=IGNORE, label_smoothing=eps, reduction="none")
    rows = (rows + z * torch.logsumexp(logits, -1) ** 2) * (lab != IGNORE).double()
    (rows.sum() / max(int((lab != IGNORE).sum()), 1)).backward()
    loss, lse, gh, gw, gb = oracle.loss_and_grads(_np(h), _np(w), _np(lab), _np(b), chunk_size=64, label_smoothing=eps,
                                                  z_loss_weight=z, dtype=np.float64, smoothing="uniform")
    np.testing.assert_allclose(gh, hd.grad.numpy(), rtol=1e-8, atol=1e-13)
    np.testing.assert_allclose(gw, wd.grad.numpy(), rtol=1e-8, atol=1e-13)
    np.testing.assert_allclose(gb, bd.grad.numpy(), rtol=1e-8, atol=1e-13)
