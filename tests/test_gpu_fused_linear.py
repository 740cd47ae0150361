"""GPU parity of the sibling fused linear-CE APIs (chronicals_amd.kernels.fused_linear_cross_entropy)
and of the remaining public classes of the drop-in module (CutCrossEntropyForward /
CutCrossEntropyBackward, reference cut_cross_entropy.py:559-808; AdaptiveCrossEntropyLoss, :1283-1372).

fused_linear_cross_entropy* / FusedLinearCrossEntropy* (reference
triton_kernels.py:2308-2817), triton_fused_linear_cross_entropy* /
TritonFusedLinearCrossEntropy* (:3147-3419, uniform-target label smoothing)
and the legacy logits-in chunked_cross_entropy (:2659-2731), through the HIP
kernels, against the CPU oracle on bf16-rounded inputs.  Tolerances: loss
within 1e-3 relative; gradients with max abs error <= 2e-2 * max|ref| and
cosine >= 0.9999.
"""
import numpy as np
import pytest
import torch

from oracle import cce_oracle as oracle
from tests.cce_common import IGNORE, assert_grad_close, assert_loss_close, bf16_exact

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _m():
    from chronicals_amd.kernels import fused_linear_cross_entropy as m
    return m


def _case(N, d, V, seed=0, bias=False, ignore_frac=0.1, oob=False):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(N, d, generator=g)
    w = torch.randn(V, d, generator=g) * 0.05
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < ignore_frac] = IGNORE
    if oob:
        lab[1] = V + 2
    b = torch.randn(V, generator=g) * 0.3 if bias else None
    return h, w, lab, b


def _dev(h, w, b, need_w=True):
    hd = h.to(DEV, torch.bfloat16).requires_grad_(True)
    wd = w.to(DEV, torch.bfloat16).requires_grad_(need_w)
    bd = None if b is None else b.to(DEV, torch.float32).requires_grad_(True)
    return hd, wd, bd


def _oracle(h, w, lab, b, eps, z, reduction, smoothing, grad_output=None):
    bn = None if b is None else b.numpy()
    return oracle.loss_and_grads(bf16_exact(h).numpy(), bf16_exact(w).numpy(), lab.numpy(), bn,
                                 label_smoothing=eps, z_loss_weight=z, reduction=reduction,
                                 grad_output=grad_output, smoothing=smoothing)


def _grads(hd, wd, bd):
    torch.cuda.synchronize()
    out = [hd.grad.float().cpu().numpy(), None if wd.grad is None else wd.grad.float().cpu().numpy(),
           None if bd is None else bd.grad.float().cpu().numpy()]
    return out


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("eps,z", [(0.1, 0.0), (0.3, 1e-3)])
def test_triton_fused_linear_uniform_smoothing(bias, reduction, eps, z):
    m = _m()
    h, w, lab, b = _case(300, 128, 5003, seed=1, bias=bias, oob=True)
    hd, wd, bd = _dev(h, w, b)
    print(f"triton_fused_linear bias={bias} reduction={reduction} eps={eps} z={z}", flush=True)
    loss = m.triton_fused_linear_cross_entropy(hd, wd, lab.to(DEV), bd, IGNORE, z, eps, reduction)
    go = torch.rand(300, generator=torch.Generator().manual_seed(2)) if reduction == "none" else None
    loss.backward(torch.ones_like(loss) if go is None else go.to(DEV))
    rl, _, gh, gw, gb = _oracle(h, w, lab, b, eps, z, reduction, "uniform", None if go is None else go.numpy())
    dh, dw, db = _grads(hd, wd, bd)
    assert_loss_close(loss.detach().cpu().numpy(), rl, "loss")
    assert_grad_close(dh, gh, "dH")
    assert_grad_close(dw, gw, "dW")
    if bias:
        assert_grad_close(db, gb, "dB")
    # the two smoothing forms really differ here
    lv = oracle.forward(bf16_exact(h).numpy(), bf16_exact(w).numpy(), lab.numpy(),
                        None if b is None else b.numpy(), label_smoothing=eps, reduction="sum")[0]
    lu = oracle.forward(bf16_exact(h).numpy(), bf16_exact(w).numpy(), lab.numpy(),
                        None if b is None else b.numpy(), label_smoothing=eps, reduction="sum", smoothing="uniform")[0]
    assert abs(float(lv) - float(lu)) > 1e-3 * abs(float(lu))


def test_triton_fused_linear_full_vocab_slice():
    # C2's d and V on a row slice, uniform smoothing with z-loss
    m = _m()
    h, w, lab, _ = _case(256, 896, 151936, seed=3)
    w = w * 0.4
    hd, wd, _ = _dev(h, w, None)
    loss = m.TritonFusedLinearCrossEntropyLoss(lse_square_scale=1e-4, label_smoothing=0.1)(hd, wd, lab.to(DEV))
    loss.backward()
    rl, _, gh, gw, _ = _oracle(h, w, lab, None, 0.1, 1e-4, "mean", "uniform")
    dh, dw, _ = _grads(hd, wd, None)
    assert_loss_close(float(loss.detach()), float(rl), "loss")
    assert_grad_close(dh, gh, "dH")
    assert_grad_close(dw, gw, "dW")
    assert m.LigerFusedLinearCrossEntropyLoss is m.TritonFusedLinearCrossEntropyLoss


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_triton_fused_linear_forward_returns_gradients(reduction):
    m = _m()
    h, w, lab, b = _case(200, 64, 3001, seed=4, bias=True)
    hd, wd, bd = _dev(h, w, b)
    wd.requires_grad_(False)
    loss, gh_, gw_, gb_ = m.triton_fused_linear_cross_entropy_forward(hd, wd, lab.to(DEV), bd, IGNORE, 1e-3, 0.2,
                                                                      reduction)
    assert gw_ is None and gb_ is not None
    # 'sum' and 'none' return the gradients of the sum (reference :3251-3263)
    ored = "mean" if reduction == "mean" else "sum"
    _, _, gh, _, gb = _oracle(h, w, lab, b, 0.2, 1e-3, ored, "uniform")
    rl = _oracle(h, w, lab, b, 0.2, 1e-3, reduction, "uniform")[0]
    torch.cuda.synchronize()
    assert_loss_close(loss.cpu().numpy(), rl, "loss")
    assert_grad_close(gh_.float().cpu().numpy(), gh, "grad_hidden")
    assert_grad_close(gb_.float().cpu().numpy(), gb, "grad_bias")


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("bias", [False, True])
def test_fused_linear_cross_entropy_loss_and_z_loss(reduction, bias):
    m = _m()
    h, w, lab, b = _case(257, 96, 4099, seed=5, bias=bias)
    hd, wd, bd = _dev(h, w, b)
    eps, z = 0.1, 1e-4
    loss, zl = m.fused_linear_cross_entropy(hd, wd, lab.to(DEV), bd, eps, z, IGNORE, 1024, reduction)
    assert not zl.requires_grad
    loss.backward(torch.ones_like(loss))
    rl, lse, gh, gw, gb = _oracle(h, w, lab, b, eps, z, reduction, "logv")
    valid = (lab != IGNORE).numpy()
    zrows = z * lse.astype(np.float64) ** 2 * valid
    rz = {"mean": zrows.sum() / max(valid.sum(), 1), "sum": zrows.sum(), "none": zrows}[reduction]
    dh, dw, db = _grads(hd, wd, bd)
    assert_loss_close(loss.detach().cpu().numpy(), rl, "loss")
    assert_loss_close(zl.cpu().numpy(), rz, "z_loss", atol=1e-9)
    assert_grad_close(dh, gh, "dH")
    assert_grad_close(dw, gw, "dW")
    if bias:
        assert_grad_close(db, gb, "dB")


def test_fused_linear_autograd_function_module_and_alias():
    m = _m()
    h, w, lab, b = _case(300, 128, 5000, seed=6, bias=True)
    hd, wd, bd = _dev(h, w, b)
    # the reference's positional order: hidden, weight, bias, labels
    loss, zl = m.FusedLinearCrossEntropyLoss(chunk_size=2048, label_smoothing=0.05)(hd, wd, bd, lab.to(DEV))
    (loss * 0.5).backward()
    rl, _, gh, gw, gb = _oracle(h, w, lab, b, 0.05, 1e-4, "mean", "logv", grad_output=np.array([0.5]))
    dh, dw, db = _grads(hd, wd, bd)
    assert_loss_close(float(loss.detach()), float(rl), "loss")
    assert_grad_close(dh, gh, "dH")
    assert_grad_close(dw, gw, "dW")
    assert_grad_close(db, gb, "dB")
    assert m.ChunkedCrossEntropyLoss is m.FusedLinearCrossEntropyLoss
    l2, z2 = m.FusedLinearCrossEntropyFunction.apply(hd, wd, bd, lab.to(DEV), 0.05, 1e-4, IGNORE, 2048)
    assert float(l2) == float(loss) and float(z2) == float(zl)


def test_fused_linear_forward_helper():
    m = _m()
    h, w, lab, b = _case(300, 64, 3000, seed=7, bias=True, oob=True)
    hd, wd, bd = _dev(h, w, b)
    lse, tgt, valid = m.fused_linear_cross_entropy_forward(hd, wd, lab.to(DEV), bd, 1024, IGNORE)
    _, rlse, rt, rvalid = oracle.forward(bf16_exact(h).numpy(), bf16_exact(w).numpy(), lab.numpy(), b.numpy())
    torch.cuda.synchronize()
    np.testing.assert_allclose(lse.cpu().numpy(), rlse, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(tgt.cpu().numpy(), rt, rtol=1e-4, atol=2e-4)
    assert np.array_equal(valid.cpu().numpy(), rvalid)
    assert float(tgt[1]) == 0.0  # out-of-range label: no target


def test_legacy_chunked_cross_entropy():
    m = _m()
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(3, 40, 32000, generator=g) * 2).to(torch.bfloat16)
    lab = torch.randint(0, 32000, (3, 40), generator=g)
    lab[0, :7] = IGNORE
    xd = x.to(DEV).requires_grad_(True)
    loss = m.chunked_cross_entropy(xd, lab.to(DEV), 8192, 0.1)
    loss.backward()
    xn = x.float().numpy().reshape(-1, 32000)
    rl, lse, valid = oracle.logits_forward(xn, lab.numpy().reshape(-1), 8192, IGNORE, 0.1, 1e-4, "mean", "logv",
                                           np.float64)
    rg = oracle.logits_backward(xn, lab.numpy().reshape(-1), lse, valid, np.ones(1), 0.1, 1e-4, "mean", "logv",
                                np.float64)
    torch.cuda.synchronize()
    assert_loss_close(float(loss.detach()), float(rl), "loss")
    assert_grad_close(xd.grad.float().cpu().numpy().reshape(rg.shape), rg, "dlogits")


def test_forward_and_backward_static_methods():
    from chronicals_amd.kernels.cut_cross_entropy import CutCrossEntropyBackward, CutCrossEntropyForward
    h, w, lab, b = _case(300, 96, 4001, seed=9, bias=True, oob=True)
    hd, wd, bd = _dev(h, w, b)
    loss, lse, tgt, valid = CutCrossEntropyForward.forward(hd, wd, lab.to(DEV), bd, 1024, IGNORE, 0.1, 1e-3)
    rl, rlse, rt, rvalid = oracle.forward(bf16_exact(h).numpy(), bf16_exact(w).numpy(), lab.numpy(), b.numpy(),
                                          label_smoothing=0.1, z_loss_weight=1e-3)
    torch.cuda.synchronize()
    assert_loss_close(float(loss), float(rl), "loss")
    np.testing.assert_allclose(lse.cpu().numpy(), rlse, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(tgt.cpu().numpy(), rt, rtol=1e-4, atol=2e-4)
    assert np.array_equal(valid.cpu().numpy(), rvalid)
    # scalar grad_output: the mean loss's gradients times it
    gh_, gw_, gb_ = CutCrossEntropyBackward.backward(hd, wd, lab.to(DEV), lse, valid, torch.tensor(2.0, device=DEV),
                                                     bd, 1024, IGNORE, 0.1, 1e-3)
    _, _, gh, gw, gb = _oracle(h, w, lab, b, 0.1, 1e-3, "mean", "logv", grad_output=np.array([2.0]))
    torch.cuda.synchronize()
    assert gh_.dtype == hd.dtype and gw_.dtype == wd.dtype and gb_.dtype == bd.dtype
    assert_grad_close(gh_.float().cpu().numpy(), gh, "dH")
    assert_grad_close(gw_.float().cpu().numpy(), gw, "dW")
    assert_grad_close(gb_.float().cpu().numpy(), gb, "dB")
    # a narrower valid mask than the labels', and a per-row grad_output (row n scaled by g[n] / n_valid)
    vm = valid.clone()
    vm[::3] = False
    go = torch.rand(300, generator=torch.Generator().manual_seed(10))
    gh_, gw_, _ = CutCrossEntropyBackward.backward(hd, wd, lab.to(DEV), lse, vm, go.to(DEV), None, 1024, IGNORE,
                                                   0.1, 1e-3)
    lab2 = lab.clone()
    lab2[~vm.cpu()] = IGNORE
    nv = int(vm.sum())
    _, _, gh, gw, _ = oracle.loss_and_grads(bf16_exact(h).numpy(), bf16_exact(w).numpy(), lab2.numpy(), None,
                                            label_smoothing=0.1, z_loss_weight=1e-3, reduction="none",
                                            grad_output=go.numpy() / nv)
    torch.cuda.synchronize()
    assert_grad_close(gh_.float().cpu().numpy(), gh, "dH per-row")
    assert_grad_close(gw_.float().cpu().numpy(), gw, "dW per-row")


@pytest.mark.parametrize("V", [5003, 40000])
@pytest.mark.parametrize("mode", ["hidden", "logits"])
def test_adaptive_cross_entropy_loss(V, mode):
    import torch.nn.functional as F
    from chronicals_amd.kernels.cut_cross_entropy import AdaptiveCrossEntropyLoss
    eps, z = 0.1, 1e-3
    h, w, lab, _ = _case(200, 64, V, seed=11)
    loss_fn = AdaptiveCrossEntropyLoss(label_smoothing=eps, z_loss_weight=z)
    small = V < loss_fn.small_vocab_threshold
    print(f"adaptive V={V} mode={mode} small={small}", flush=True)
    if mode == "hidden":
        hd, wd, _ = _dev(h, w, None)
        loss = loss_fn(hd, wd, lab.to(DEV))
        loss.backward()
        if small:
            # torch's CrossEntropyLoss over the logits (uniform smoothing, no z-loss)
            rl, _, gh, gw, _ = _oracle(h, w, lab, None, eps, 0.0, "mean", "uniform")
        else:
            rl, _, gh, gw, _ = _oracle(h, w, lab, None, eps, z, "mean", "logv")
        dh, dw, _ = _grads(hd, wd, None)
        assert_loss_close(float(loss.detach()), float(rl), "loss")
        assert_grad_close(dh, gh, "dH")
        assert_grad_close(dw, gw, "dW")
    else:
        x = (bf16_exact(h) @ bf16_exact(w).t()).to(torch.bfloat16)
        xd = x.to(DEV).requires_grad_(True)
        loss = loss_fn(xd, lab.to(DEV))
        loss.backward()
        xr = x.double().requires_grad_(True)
        if small:
            ref = F.cross_entropy(xr, lab, ignore_index=IGNORE, label_smoothing=eps)
        else:
            valid = lab != IGNORE
            lse_r = torch.logsumexp(xr, -1)
            t = xr.gather(1, torch.where(valid, lab, 0)[:, None])[:, 0]
            rows = ((1 - eps) * (lse_r - t) + eps * np.log(V) + z * lse_r ** 2) * valid
            ref = rows.sum() / valid.sum()
        (rg,) = torch.autograd.grad(ref, xr)
        torch.cuda.synchronize()
        assert_loss_close(float(loss.detach()), float(ref), "loss")
        assert_grad_close(xd.grad.float().cpu().numpy(), rg.numpy(), "dlogits")
