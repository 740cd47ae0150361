"""GPU parity of the logits-in cross-entropy (cce_logits_forward / _backward).

The HIP row kernels, called through the drop-in APIs
(chunked_cross_entropy_loss, liger_cross_entropy*, fused_cross_entropy) and
through the torch.library ops, against the CPU oracle
(oracle.cce_oracle.logits_forward / logits_backward, float64) on the same
seeded inputs; at the full C2 shape against a float64-accumulated closed form
on the GPU.  Tolerances: loss within 1e-3 relative, lse within 2e-5
relative; gradients with max abs error <= 2e-2 * max|ref| and cosine >=
0.9999 (tests/cce_common.py), tighter for fp32 logits.
"""
import math

import numpy as np
import pytest
import torch

from oracle import cce_oracle as oracle
from tests.cce_common import IGNORE, assert_grad_close, assert_loss_close, grad_report

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _mod():
    from chronicals_amd.kernels import logits_cross_entropy as m
    return m


def _case(N, V, dtype, seed=0, ignore_frac=0.1, oob=False, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(N, V, generator=g) * scale).to(dtype)
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < ignore_frac] = IGNORE
    if oob and N > 3:
        lab[1] = V + 3
        lab[2] = -5
    return x, lab


def oracle_ref(x, lab, eps=0.0, z=0.0, reduction="mean", smoothing="logv", grad_output=None):
    xn = x.float().numpy().reshape(-1, x.shape[-1])
    ln = lab.numpy().reshape(-1)
    loss, lse, valid = oracle.logits_forward(xn, ln, 8192, IGNORE, eps, z, reduction, smoothing, np.float64)
    if grad_output is None:
        grad_output = np.ones(ln.size) if reduction == "none" else np.ones(1)
    g = oracle.logits_backward(xn, ln, lse, valid, grad_output, eps, z, reduction, smoothing, np.float64)
    return loss, lse, g


def _sync_np(t):
    torch.cuda.synchronize()
    return t.detach().float().cpu().numpy()


def chunked_hip(x, lab, eps=0.0, z=0.0, reduction="mean", grad_output=None, labels_dtype=torch.int64):
    m = _mod()
    xd = x.to(DEV).requires_grad_(True)
    loss = m.chunked_cross_entropy_loss(xd, lab.to(DEV, labels_dtype), 8192, IGNORE, eps, z, reduction=reduction)
    go = torch.ones_like(loss) if grad_output is None else torch.as_tensor(grad_output, dtype=torch.float32,
                                                                            device=DEV).reshape(loss.shape)
    loss.backward(go)
    return _sync_np(loss), xd.grad


def _check_grad(got_t, ref, dtype, what):
    got = _sync_np(got_t).reshape(ref.shape)
    if ref.size and np.abs(ref).max() < 1e-6:
        # V = 1: the exact gradient is the 1e-10 of log(s + 1e-10), below fp32 resolution
        assert np.abs(got - ref).max() <= 1e-6, f"{what}: {grad_report(got, ref)}"
        return
    assert_grad_close(got, ref, what)
    if dtype == torch.float32:
        r = grad_report(got, ref)
        assert r["frac"] <= 1e-4 and r["cos"] >= 1 - 1e-9, f"{what}: fp32 path {r}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("N,V", [(37, 1000), (64, 50257), (5, 7), (3, 1), (129, 151936)])
def test_chunked_matches_oracle(dtype, N, V):
    x, lab = _case(N, V, dtype, seed=N + V, oob=True)
    if V == 1:
        lab = torch.where(lab == IGNORE, lab, torch.zeros_like(lab))
    print(f"chunked dtype={dtype} N={N} V={V}", flush=True)
    loss, gx = chunked_hip(x, lab)
    rl, _, rg = oracle_ref(x, lab)
    assert_loss_close(loss, rl, "loss")
    assert gx.dtype == dtype and gx.shape == x.shape
    _check_grad(gx, rg, dtype, "dlogits")


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("eps,z", [(0.0, 0.0), (0.1, 1e-4), (0.3, 1e-2)])
def test_chunked_reductions_smoothing_zloss(reduction, eps, z):
    x, lab = _case(300, 5003, torch.bfloat16, seed=11, ignore_frac=0.25)
    go = None
    if reduction == "none":
        go = torch.rand(300, generator=torch.Generator().manual_seed(3)).numpy()
    print(f"chunked reduction={reduction} eps={eps} z={z}", flush=True)
    loss, gx = chunked_hip(x, lab, eps, z, reduction, go)
    rl, _, rg = oracle_ref(x, lab, eps, z, reduction, "logv", go)
    assert_loss_close(loss, rl, "loss")
    _check_grad(gx, rg, torch.bfloat16, "dlogits")


def test_chunked_3d_int32_labels_and_module():
    m = _mod()
    x, lab = _case(4 * 75, 32000, torch.bfloat16, seed=5)
    x3, lab3 = x.view(4, 75, 32000), lab.view(4, 75)
    loss, gx = chunked_hip(x3, lab3, 0.1, 1e-3, labels_dtype=torch.int32)
    rl, _, rg = oracle_ref(x, lab, 0.1, 1e-3)
    assert_loss_close(loss, rl, "loss")
    assert gx.shape == (4, 75, 32000)
    _check_grad(gx, rg.reshape(4, 75, 32000), torch.bfloat16, "dlogits")
    mod_loss = m.ChunkedCrossEntropyLoss(label_smoothing=0.1, z_loss_weight=1e-3)(x3.to(DEV), lab3.to(DEV))
    assert float(mod_loss) == float(loss)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_strided_rows(dtype):
    # logits a column slice of a wider buffer: row stride > V, rows not 16-byte aligned alike
    N, V, W = 96, 10001, 10240
    wide, lab = _case(N, W, dtype, seed=9)
    x = wide.to(DEV)[:, 3:3 + V]
    lab = lab.clamp(max=V - 1)
    assert x.stride(0) == W and x.stride(1) == 1
    m = _mod()
    xl = x.detach().requires_grad_(True)
    loss = m.chunked_cross_entropy_loss(xl, lab.to(DEV), label_smoothing=0.05)
    loss.backward()
    rl, _, rg = oracle_ref(wide[:, 3:3 + V].contiguous(), lab, 0.05)
    assert_loss_close(_sync_np(loss), rl, "loss")
    _check_grad(xl.grad, rg, dtype, "dlogits")


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("eps,z", [(0.0, 0.0), (0.2, 1e-3)])
def test_liger_autograd_matches_oracle(reduction, eps, z):
    m = _mod()
    x, lab = _case(200, 32768, torch.bfloat16, seed=21, oob=True)
    xd = x.to(DEV).requires_grad_(True)
    print(f"liger reduction={reduction} eps={eps} z={z}", flush=True)
    loss = m.liger_cross_entropy(xd, lab.to(DEV), IGNORE, z, eps, reduction)
    go = torch.rand(200, generator=torch.Generator().manual_seed(4)).numpy() if reduction == "none" else None
    loss.backward(torch.ones_like(loss) if go is None else torch.as_tensor(go, dtype=torch.float32, device=DEV))
    rl, _, rg = oracle_ref(x, lab, eps, z, reduction, "uniform", go)
    assert_loss_close(_sync_np(loss), rl, "loss")
    _check_grad(xd.grad, rg, torch.bfloat16, "dlogits")


@pytest.mark.parametrize("reduction", ["mean", "none"])
def test_liger_forward_overwrites_logits_with_gradient(reduction):
    m = _mod()
    x, lab = _case(3 * 50, 50257, torch.float32, seed=23)
    xd = x.view(3, 50, 50257).to(DEV).clone()
    ptr = xd.data_ptr()
    loss, grads = m.liger_cross_entropy_forward(xd, lab.view(3, 50).to(DEV), IGNORE, 1e-4, 0.1, reduction)
    assert grads.data_ptr() == ptr and grads.shape == (150, 50257)
    rl, _, rg = oracle_ref(x, lab, 0.1, 1e-4, reduction, "uniform")
    # 'none' gradients are not divided by n_valid, as the reference kernel stores them
    if reduction == "none":
        rg = oracle.logits_backward(x.numpy(), lab.numpy(),
                                    oracle.logits_forward(x.numpy(), lab.numpy(), 8192, IGNORE, 0.1, 1e-4, "sum",
                                                          "uniform", np.float64)[1],
                                    (lab != IGNORE).numpy(), np.ones(1), 0.1, 1e-4, "sum", "uniform", np.float64)
    assert_loss_close(_sync_np(loss), rl, "loss")
    _check_grad(grads, rg, torch.float32, "in-place dlogits")
    scaled = m.liger_cross_entropy_backward(grads, torch.tensor(0.5, device=DEV))
    _check_grad(scaled, 0.5 * rg, torch.float32, "scaled dlogits")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_cross_entropy_mean_loss_and_fp32_row_gradients(dtype):
    m = _mod()
    x, lab = _case(2 * 64, 50257, dtype, seed=31)
    loss, dl = m.fused_cross_entropy(x.view(2, 64, 50257).to(DEV), lab.view(2, 64).to(DEV), 0.1, 1e-4, IGNORE)
    assert dl.dtype == torch.float32 and dl.shape == (2, 64, 50257)
    rl, lse, _ = oracle_ref(x, lab, 0.1, 1e-4, "mean", "uniform")
    valid = (lab != IGNORE).numpy()
    rg = oracle.logits_backward(x.float().numpy(), lab.numpy(), lse, valid, np.ones(1), 0.1, 1e-4, "sum",
                                "uniform", np.float64)
    assert_loss_close(_sync_np(loss), rl, "loss")
    _check_grad(dl, rg.reshape(2, 64, 50257), torch.float32, "dlogits")


def test_all_ignored_and_empty():
    m = _mod()
    x = torch.randn(16, 3000).to(DEV, torch.bfloat16).requires_grad_(True)
    lab = torch.full((16,), IGNORE, device=DEV)
    loss = m.chunked_cross_entropy_loss(x, lab, label_smoothing=0.1, z_loss_weight=0.01)
    loss.backward()
    assert float(loss) == 0.0 and not x.grad.float().abs().sum().item()
    e = torch.empty(0, 3000, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    le = m.chunked_cross_entropy_loss(e, torch.empty(0, dtype=torch.long, device=DEV))
    le.backward()
    assert float(le) == 0.0 and e.grad.shape == (0, 3000)
    ln = m.chunked_cross_entropy_loss(e, torch.empty(0, dtype=torch.long, device=DEV), reduction="none")
    assert ln.shape == (0,)


def test_deterministic():
    m = _mod()
    x, lab = _case(512, 151936, torch.bfloat16, seed=41)
    xd, ld = x.to(DEV), lab.to(DEV)
    outs = []
    for _ in range(2):
        xr = xd.detach().requires_grad_(True)
        loss = m.chunked_cross_entropy_loss(xr, ld, label_smoothing=0.1, z_loss_weight=1e-4)
        loss.backward()
        torch.cuda.synchronize()
        outs.append((loss.detach().clone(), xr.grad.clone()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])


def test_side_streams_concurrent_no_host_sync():
    """The logits-in ops launch on the caller's current stream and never
    synchronise with the host: two problems run concurrently on two side
    streams under torch's sync debug mode "error", each after a bounded spin
    and a fresh input copy on its own stream, and match the default-stream
    results bitwise."""
    m = _mod()
    cases = [_case(300, 50257, torch.bfloat16, seed=43), _case(700, 32000, torch.float32, seed=44)]
    refs = []
    for x, lab in cases:
        xr = x.to(DEV).requires_grad_(True)
        loss = m.chunked_cross_entropy_loss(xr, lab.to(DEV), label_smoothing=0.1, z_loss_weight=1e-4)
        loss.backward()
        torch.cuda.synchronize()
        refs.append((loss.detach().clone(), xr.grad.clone()))
    sources = [(x.to(DEV), lab.to(DEV)) for x, lab in cases]
    main = torch.cuda.current_stream()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    torch.cuda.set_sync_debug_mode("error")
    try:
        for s, (x0, l0) in zip(streams, sources):
            s.wait_stream(main)
            with torch.cuda.stream(s):
                torch.cuda._sleep(20_000_000)  # about 10 ms of spinning on this stream
                xr = x0.clone().requires_grad_(True)
                loss = m.chunked_cross_entropy_loss(xr, l0.clone(), label_smoothing=0.1, z_loss_weight=1e-4)
                loss.backward()
                outs.append((loss, xr))
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    for i, ((rl, rg), (loss, xr)) in enumerate(zip(refs, outs)):
        assert torch.equal(loss.detach(), rl), f"case {i} loss"
        assert torch.equal(xr.grad, rg), f"case {i} grad"


def test_full_size_C2_logits_against_gpu_closed_form():
    # N x V of C2 (16384 x 151936 bf16 logits, 5 GB): float64-accumulated closed form on the GPU, by row blocks
    m = _mod()
    N, V = 16384, 151936
    g = torch.Generator(device=DEV).manual_seed(0)
    x = (torch.randn(N, V, generator=g, device=DEV) * 3.0).to(torch.bfloat16)
    lab = torch.randint(0, V, (N,), generator=g, device=DEV)
    lab[torch.rand(N, generator=g, device=DEV) < 0.05] = IGNORE
    eps, z = 0.1, 1e-4
    xr = x.detach().requires_grad_(True)
    print("C2 logits: HIP forward/backward", flush=True)
    loss = m.chunked_cross_entropy_loss(xr, lab, label_smoothing=eps, z_loss_weight=z)
    loss.backward()
    torch.cuda.synchronize()
    valid = lab != IGNORE
    nv = max(int(valid.sum()), 1)
    total = torch.zeros((), dtype=torch.float64, device=DEV)
    worst_frac, cos_num, cos_a, cos_b, gmax = 0.0, 0.0, 0.0, 0.0, 0.0
    for r0 in range(0, N, 1024):
        xb = x[r0:r0 + 1024].double()
        lb = lab[r0:r0 + 1024]
        vb = valid[r0:r0 + 1024]
        lse = torch.logsumexp(xb, dim=-1)
        t = xb.gather(1, torch.where(vb, lb, 0)[:, None])[:, 0]
        row = ((1 - eps) * (lse - t) + eps * math.log(V) + z * lse * lse) * vb.double()
        total += row.sum()
        p = torch.exp(xb - lse[:, None])
        gr = ((1 - eps) + 2 * z * lse[:, None]) * p
        idx = torch.nonzero(vb)[:, 0]
        gr[idx, lb[idx]] -= (1 - eps)
        gr = gr * vb.double()[:, None] / nv
        got = xr.grad[r0:r0 + 1024].double()
        gmax = max(gmax, float(gr.abs().max()))
        worst_frac = max(worst_frac, float((got - gr).abs().max()))
        cos_num += float((got * gr).sum())
        cos_a += float((got * got).sum())
        cos_b += float((gr * gr).sum())
    assert_loss_close(float(loss), float(total / nv), "C2 loss")
    assert worst_frac <= 2e-2 * gmax, (worst_frac, gmax)
    assert cos_num / math.sqrt(cos_a * cos_b) >= 0.9999


def test_custom_ops_opcheck():
    from torch.library import opcheck
    from chronicals_amd import _lib
    x, lab = _case(64, 1000, torch.bfloat16, seed=51)
    xd, ld = x.to(DEV), lab.to(DEV)
    args = (xd, ld, IGNORE, 0.1, 1e-4, _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_REDUCTION_MEAN)
    opcheck(torch.ops.chronicals_hip.ce_logits_fwd.default, args)
    loss, lse, nv = torch.ops.chronicals_hip.ce_logits_fwd(*args)
    go = torch.ones(1, device=DEV)
    for f32 in (False, True):
        opcheck(torch.ops.chronicals_hip.ce_logits_bwd.default,
                (go, xd, ld, lse, nv, IGNORE, 0.1, 1e-4, _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_REDUCTION_MEAN, f32))
    opcheck(torch.ops.chronicals_hip.ce_logits_bwd_.default,
            (go, xd.clone(), ld, lse, nv, IGNORE, 0.1, 1e-4, _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_REDUCTION_MEAN))


def test_torch_compile_fullgraph():
    m = _mod()
    x, lab = _case(128, 32000, torch.bfloat16, seed=61)

    def f(logits, labels):
        return m.chunked_cross_entropy_loss(logits * 1.0, labels, label_smoothing=0.1)

    cf = torch.compile(f, fullgraph=True)
    x1 = x.to(DEV).requires_grad_(True)
    x2 = x.to(DEV).requires_grad_(True)
    l1 = f(x1, lab.to(DEV))
    l1.backward()
    l2 = cf(x2, lab.to(DEV))
    l2.backward()
    torch.cuda.synchronize()
    assert torch.allclose(l1, l2, rtol=1e-6)
    assert torch.equal(x1.grad, x2.grad)


def test_overlapping_and_single_row_views_are_copied():
    m = _mod()
    row = torch.randn(1, 4099).to(DEV, torch.bfloat16)
    lab = torch.tensor([7, 4000, 12], device=DEV)
    x = row.expand(3, 4099)  # row stride 0
    loss = m.chunked_cross_entropy_loss(x, lab)
    ref = torch.nn.functional.cross_entropy(row.float().expand(3, 4099), lab)
    assert_loss_close(float(loss), float(ref), "expanded rows")
    t = torch.randn(4099, 2).to(DEV, torch.bfloat16)
    xt = t[:, :1].t()  # one row, last-dimension stride 2
    l1 = m.chunked_cross_entropy_loss(xt, lab[:1])
    r1 = torch.nn.functional.cross_entropy(xt.float(), lab[:1])
    assert_loss_close(float(l1), float(r1), "strided single row")


# ---------------------------------------------------------------------------
# cce_logits_forward_backward: loss and gradient in one kernel
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype,f32", [(torch.bfloat16, False), (torch.bfloat16, True), (torch.float16, True),
                                       (torch.float32, True)])
@pytest.mark.parametrize("form", ["logv", "uniform"])
@pytest.mark.parametrize("reduction,grad_mean", [("mean", True), ("mean", False), ("sum", False), ("none", False)])
def test_fused_loss_and_gradient_kernel(dtype, f32, form, reduction, grad_mean):
    from chronicals_amd import _lib
    # N above the rows kept in flight (2 per CU), so workgroups take several rows; odd V
    N, V = 3000, 20011
    x, lab = _case(N, V, dtype, seed=71, oob=True)
    code = _lib.CCE_SMOOTH_LOGV if form == "logv" else _lib.CCE_SMOOTH_UNIFORM
    red = _lib.REDUCTIONS[reduction]
    print(f"fused kernel dtype={dtype} f32={f32} form={form} reduction={reduction} grad_mean={grad_mean}", flush=True)
    loss, lse, nv, dx = torch.ops.chronicals_hip.ce_logits_fwd_bwd(x.to(DEV), lab.to(DEV), IGNORE, 0.1, 1e-3, code,
                                                                   red, grad_mean, f32)
    rl, rlse, _ = oracle_ref(x, lab, 0.1, 1e-3, reduction, form)
    gred = "mean" if grad_mean else "sum"
    _, _, rg = oracle_ref(x, lab, 0.1, 1e-3, gred, form)
    torch.cuda.synchronize()
    assert dx.dtype == (torch.float32 if f32 else dtype)
    assert int(nv) == int((lab != IGNORE).sum())
    np.testing.assert_allclose(lse.cpu().numpy(), rlse, rtol=2e-5, atol=2e-5)
    assert_loss_close(loss.cpu().numpy().reshape(np.shape(rl)), rl, "loss")
    _check_grad(dx, rg, torch.float32 if dtype == torch.float32 else torch.bfloat16, "dlogits")


def test_fused_kernel_in_place_matches_out_of_place_and_two_kernel_path():
    from chronicals_amd import _lib
    N, V = 1500, 32768
    x, lab = _case(N, V, torch.bfloat16, seed=72)
    xd, ld = x.to(DEV), lab.to(DEV)
    l1, _, _, g1 = torch.ops.chronicals_hip.ce_logits_fwd_bwd(xd, ld, IGNORE, 0.2, 0.0, _lib.CCE_SMOOTH_UNIFORM,
                                                              _lib.CCE_REDUCTION_MEAN, True, False)
    xi = xd.clone()
    l2, _, _ = torch.ops.chronicals_hip.ce_logits_fwd_bwd_(xi, ld, IGNORE, 0.2, 0.0, _lib.CCE_SMOOTH_UNIFORM,
                                                           _lib.CCE_REDUCTION_MEAN, True)
    torch.cuda.synchronize()
    assert torch.equal(l1, l2) and torch.equal(g1, xi)
    # the same numbers as forward + backward kernels (different reduction trees: ulp-level differences)
    l3, lse3, nv3 = torch.ops.chronicals_hip.ce_logits_fwd(xd, ld, IGNORE, 0.2, 0.0, _lib.CCE_SMOOTH_UNIFORM,
                                                           _lib.CCE_REDUCTION_MEAN)
    g3 = torch.ops.chronicals_hip.ce_logits_bwd(torch.ones(1, device=DEV), xd, ld, lse3, nv3, IGNORE, 0.2, 0.0,
                                                _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_REDUCTION_MEAN, False)
    torch.cuda.synchronize()
    assert_loss_close(float(l1), float(l3), "loss", rtol=1e-6)
    r = grad_report(g1.float().cpu().numpy(), g3.float().cpu().numpy())
    assert r["frac"] <= 1e-2 and r["cos"] >= 1 - 1e-6, r


def test_fused_kernel_ops_opcheck_and_determinism():
    from torch.library import opcheck
    from chronicals_amd import _lib
    x, lab = _case(600, 5000, torch.bfloat16, seed=73)
    xd, ld = x.to(DEV), lab.to(DEV)
    for f32 in (False, True):
        opcheck(torch.ops.chronicals_hip.ce_logits_fwd_bwd.default,
                (xd, ld, IGNORE, 0.1, 1e-4, _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_REDUCTION_MEAN, True, f32))
    opcheck(torch.ops.chronicals_hip.ce_logits_fwd_bwd_.default,
            (xd.clone(), ld, IGNORE, 0.1, 1e-4, _lib.CCE_SMOOTH_LOGV, _lib.CCE_REDUCTION_SUM, False))
    a = torch.ops.chronicals_hip.ce_logits_fwd_bwd(xd, ld, IGNORE, 0.1, 1e-4, 1, 1, True, False)
    b = torch.ops.chronicals_hip.ce_logits_fwd_bwd(xd, ld, IGNORE, 0.1, 1e-4, 1, 1, True, False)
    torch.cuda.synchronize()
    assert all(torch.equal(p, q) for p, q in zip(a, b))


def test_fused_kernel_all_ignored_and_empty():
    from chronicals_amd import _lib
    x = torch.randn(700, 3000).to(DEV, torch.bfloat16)
    lab = torch.full((700,), IGNORE, device=DEV)
    loss, _, nv, g = torch.ops.chronicals_hip.ce_logits_fwd_bwd(x, lab, IGNORE, 0.1, 1e-2, 1, 1, True, True)
    torch.cuda.synchronize()
    assert float(loss) == 0.0 and int(nv) == 0 and not g.abs().sum().item()
    e = torch.empty(0, 3000, device=DEV, dtype=torch.bfloat16)
    loss, _, nv, g = torch.ops.chronicals_hip.ce_logits_fwd_bwd(e, torch.empty(0, dtype=torch.long, device=DEV),
                                                                IGNORE, 0.0, 0.0, 0, 1, True, False)
    torch.cuda.synchronize()
    assert float(loss) == 0.0 and int(nv) == 0 and g.shape == (0, 3000)


@pytest.mark.parametrize("scale", [300.0, 3000.0])
def test_extreme_logit_magnitudes(scale):
    # logits in the thousands: the online max keeps exp2 in range; float64 closed form as reference
    m = _mod()
    x, lab = _case(257, 4099, torch.float32, seed=81, scale=scale)
    xd = x.to(DEV).requires_grad_(True)
    loss = m.chunked_cross_entropy_loss(xd, lab.to(DEV), label_smoothing=0.1, z_loss_weight=1e-6)
    loss.backward()
    rl, _, rg = oracle_ref(x, lab, 0.1, 1e-6)
    assert np.isfinite(float(loss.detach())) and torch.isfinite(xd.grad).all()
    assert_loss_close(float(loss.detach()), float(rl), "loss")
    _check_grad(xd.grad, rg, torch.bfloat16, "dlogits")
