"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Inputs are rounded to bf16 before either side sees them (the kernels compute
in bf16 with fp32 accumulation), so the comparison measures the kernels'
own error.  Tolerances (tests/cce_common.py): loss within 1e-3 relative;
gradients with max abs error <= 2e-2 * max|ref| and cosine >= 0.9999.
Full-size configurations use a materialised fp32 torch reference on the GPU.
"""
import os

import numpy as np
import pytest
import torch

from oracle import cce_oracle as oracle
from tests.cce_common import (CONFIGS, IGNORE, assert_grad_close, assert_grad_close_torch, assert_loss_close,
                              bf16_exact, grad_report_torch, make_inputs, torch_reference_rows)

pytestmark = pytest.mark.gpu


def _cce():
    from chronicals_amd.kernels.cut_cross_entropy import cut_cross_entropy
    return cut_cross_entropy


def run_hip(dev, h, w, lab, b=None, chunk=8192, eps=0.0, z=0.0, reduction="mean", grad_output=None,
            need_dh=True, need_dw=True, need_db=True, hdtype=torch.bfloat16, wdtype=torch.bfloat16):
    hd = h.detach().to(dev, hdtype).requires_grad_(need_dh)
    wd = w.detach().to(dev, wdtype).requires_grad_(need_dw)
    bd = None if b is None else b.detach().to(dev, torch.float32).requires_grad_(need_db)
    ld = lab.to(dev)
    loss = _cce()(hd, wd, ld, bd, chunk, IGNORE, eps, z, reduction=reduction)
    if need_dh or need_dw or (b is not None and need_db):
        if reduction == "none":
            go = torch.ones_like(loss) if grad_output is None else grad_output.to(dev).reshape(loss.shape)
            loss.backward(go)
        else:
            loss.backward(None if grad_output is None else torch.tensor(float(grad_output), device=dev))
    torch.cuda.synchronize()
    out = {"loss": loss.detach().float().cpu().numpy()}
    out["dh"] = None if not need_dh else hd.grad.float().cpu().numpy()
    out["dw"] = None if not need_dw else wd.grad.float().cpu().numpy()
    out["db"] = None if (b is None or not need_db) else bd.grad.float().cpu().numpy()
    return out


def run_oracle(h, w, lab, b=None, chunk=8192, eps=0.0, z=0.0, reduction="mean", grad_output=None):
    hn = bf16_exact(h).numpy().reshape(-1, h.shape[-1])
    wn = bf16_exact(w).numpy()
    bn = None if b is None else b.float().numpy()
    go = None
    if grad_output is not None:
        go = np.asarray(grad_output.numpy() if torch.is_tensor(grad_output) else [grad_output], np.float64)
    loss, lse, gh, gw, gb = oracle.loss_and_grads(hn, wn, lab.numpy().reshape(-1), bn, chunk_size=chunk,
                                                  label_smoothing=eps, z_loss_weight=z, reduction=reduction,
                                                  grad_output=go)
    return {"loss": np.asarray(loss).reshape(np.asarray(lab).shape) if reduction == "none" else loss,
            "lse": lse, "dh": gh, "dw": gw, "db": gb}


def compare(got, ref, tag):
    assert_loss_close(got["loss"], ref["loss"], f"{tag} loss")
    for k in ("dh", "dw", "db"):
        if got.get(k) is not None and ref.get(k) is not None:
            assert_grad_close(got[k].reshape(ref[k].shape), ref[k], f"{tag} {k}")


def _rand_case(N, d, V, seed=0, ignore_frac=0.1, bias=False, wscale=0.05):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(N, d, generator=g)
    w = torch.randn(V, d, generator=g) * wscale
    lab = torch.randint(0, V, (N,), generator=g)
    if N:
        lab[torch.rand(N, generator=g) < ignore_frac] = IGNORE
    b = torch.randn(V, generator=g) * 0.1 if bias else None
    return h, w, lab, b


@pytest.mark.parametrize("N,d,V,chunk", [
    (256, 64, 256, 8192),      # one tile
    (1, 8, 1, 8192),           # smallest problem
    (3, 16, 7, 8192),
    (255, 72, 257, 256),       # ragged rows / columns, two bands
    (257, 136, 1000, 512),     # d not a multiple of 64, ragged bands
    (600, 128, 5000, 1024),
    (513, 264, 3001, 8192),
    (300, 192, 2100, 512),     # d % 256 > 128: one padded 256-wide dH column tile
    (333, 320, 1500, 768),     # d = 256 + 64: 256-wide dH tile plus a 128-wide tail tile
])
def test_ragged_shapes(gpu, N, d, V, chunk):
    print(f"case N={N} d={d} V={V} chunk={chunk}", flush=True)
    h, w, lab, _ = _rand_case(N, d, V, seed=N + V)
    compare(run_hip(gpu, h, w, lab, chunk=chunk), run_oracle(h, w, lab, chunk=chunk), f"N{N}d{d}V{V}")


@pytest.mark.parametrize("N,d,V,chunk,hdtype,reduction,ignore_frac", [
    # 9 dH tiles: 15 K splits; a partial first band and two full ones (accumulator modes 1, 2, 3);
    # fp32 gradients; per-row grad_output
    (700, 768, 20000, 8192, torch.float32, "none", 0.1),
    # d = 256 + 64: the 128-wide tail tile is split too; most rows ignored (one live row tile of three)
    (600, 320, 9000, 4096, torch.bfloat16, "mean", 0.7),
    # one band (mode 0: straight to the output; the band is 3072 wide): 6 splits of 512 columns, the last shorter
    (130, 512, 3000, 8192, torch.bfloat16, "sum", 0.1),
    # V = 8 * 8192 + 40: 9 bands of 8192 (256 rows are not widened); the 40-column first band is left with a
    # single split and still writes partials
    (256, 768, 65576, 8192, torch.bfloat16, "mean", 0.1),
    # 1100 rows widen chunk 1024 to 3072-column bands: 7 bands; d = 128 is one 128-wide tail tile (5 dH tiles,
    # 6 K splits: the reduction rides in the next band's launch); 30% of the rows ignored
    (1100, 128, 20000, 1024, torch.bfloat16, "mean", 0.3),
    # 1300 rows widen chunk 2048 to 4096: 3 bands (a 808-column first band); 6 dH tiles of 256 columns, 8 splits
    (1300, 256, 9000, 2048, torch.float32, "sum", 0.1),
])
def test_small_batch_split_dh(gpu, N, d, V, chunk, hdtype, reduction, ignore_frac):
    """With few 256-row tiles the banded dH splits each band's K over several
    workgroups (fp32 partials, then a fixed-order reduction that applies the
    band's accumulator mode); against the oracle, and bitwise repeatable."""
    print(f"case split dH N={N} d={d} V={V} chunk={chunk} {hdtype} {reduction}", flush=True)
    h, w, lab, _ = _rand_case(N, d, V, seed=N + d, ignore_frac=ignore_frac)
    go = torch.rand(N, generator=torch.Generator().manual_seed(4)) if reduction == "none" else None
    got = run_hip(gpu, h, w, lab, chunk=chunk, reduction=reduction, grad_output=go, hdtype=hdtype)
    compare(got, run_oracle(h, w, lab, chunk=chunk, reduction=reduction, grad_output=go), f"split N{N}d{d}")
    again = run_hip(gpu, h, w, lab, chunk=chunk, reduction=reduction, grad_output=go, hdtype=hdtype)
    assert np.array_equal(got["dh"], again["dh"]) and np.array_equal(got["dw"], again["dw"])


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("bias", [False, True])
def test_reductions_and_bias(gpu, reduction, bias):
    print(f"case reduction={reduction} bias={bias}", flush=True)
    h, w, lab, b = _rand_case(300, 96, 2000, seed=11, bias=bias)
    go = torch.rand(300, generator=torch.Generator().manual_seed(3)) if reduction == "none" else 0.7
    got = run_hip(gpu, h, w, lab, b, chunk=768, reduction=reduction, grad_output=go)
    ref = run_oracle(h, w, lab, b, chunk=768, reduction=reduction, grad_output=go)
    compare(got, ref, f"{reduction}/bias={bias}")


@pytest.mark.parametrize("eps,z", [(0.1, 0.0), (0.0, 1e-3), (0.1, 1e-4)])
def test_label_smoothing_and_zloss(gpu, eps, z):
    print(f"case eps={eps} z={z}", flush=True)
    h, w, lab, b = _rand_case(400, 64, 3000, seed=5, bias=True)
    compare(run_hip(gpu, h, w, lab, b, chunk=1024, eps=eps, z=z),
            run_oracle(h, w, lab, b, chunk=1024, eps=eps, z=z), f"eps{eps}z{z}")


def test_out_of_range_labels(gpu):
    h, w, lab, _ = _rand_case(64, 32, 500, seed=2)
    lab[3] = 500
    lab[4] = 10**6
    lab[5] = -5
    compare(run_hip(gpu, h, w, lab), run_oracle(h, w, lab), "oob")


def test_all_ignored(gpu):
    h, w, lab, b = _rand_case(100, 64, 700, seed=9, bias=True)
    lab[:] = IGNORE
    got = run_hip(gpu, h, w, lab, b)
    assert float(got["loss"]) == 0.0
    assert not np.any(got["dh"]) and not np.any(got["dw"]) and not np.any(got["db"])


@pytest.mark.parametrize("reduction,bias,hdtype", [("mean", True, torch.bfloat16), ("none", False, torch.float32),
                                                    ("sum", True, torch.float32)])
def test_ignored_row_tiles_are_skipped(gpu, reduction, bias, hdtype):
    # The banded backward compacts the labelled rows to the front and skips
    # the 256-row tiles past them: 400 labelled rows of 1100 leave 2 of 5 row
    # tiles live.  The ignored rows' dH must still be exactly zero.  V = 9500
    # keeps 4 bands (1100 rows widen chunk 1024 to 3072-column bands), so the
    # accumulator modes 1, 2 and 3 all run on the compacted rows.
    print(f"case compaction reduction={reduction} bias={bias} hdtype={hdtype}", flush=True)
    h, w, lab, b = _rand_case(1100, 128, 9500, seed=21, ignore_frac=0.0, bias=bias)
    g = torch.Generator().manual_seed(4)
    lab[torch.randperm(1100, generator=g)[:700]] = IGNORE
    go = torch.rand(1100, generator=g) if reduction == "none" else 1.3
    got = run_hip(gpu, h, w, lab, b, chunk=1024, reduction=reduction, grad_output=go, hdtype=hdtype)
    ref = run_oracle(h, w, lab, b, chunk=1024, reduction=reduction, grad_output=go)
    compare(got, ref, f"compaction {reduction}")
    ign = (lab == IGNORE).numpy()
    assert not np.any(got["dh"][ign])


def test_all_ignored_many_row_tiles(gpu):
    h, w, lab, b = _rand_case(1000, 64, 700, seed=19, bias=True)
    lab[:] = IGNORE
    got = run_hip(gpu, h, w, lab, b, chunk=256)
    assert float(got["loss"]) == 0.0
    assert not np.any(got["dh"]) and not np.any(got["dw"]) and not np.any(got["db"])


def test_labelled_rows_at_the_end(gpu):
    # the labelled rows sit in the last row tile; compaction moves them to the first
    h, w, lab, _ = _rand_case(900, 192, 2500, seed=23, ignore_frac=0.0)
    lab[:850] = IGNORE
    compare(run_hip(gpu, h, w, lab, chunk=512), run_oracle(h, w, lab, chunk=512), "tail rows")


@pytest.mark.parametrize("d", [128, 72])
def test_forward_lse_labelled_rows(gpu, d):
    """CCE_LSE_LABELLED_ROWS: the same loss and n_valid as CCE_LSE_ALL_ROWS, the
    same lse / target on labelled rows, 0 on ignored rows (d = 128 compacts
    the rows; d = 72 runs the register-staged GEMM over every row).  V = 9500
    gives the autograd check 4 backward bands of 3072 columns."""
    from chronicals_amd import _lib
    print(f"case lse_rows d={d}", flush=True)
    h, w, lab, b = _rand_case(1100, d, 9500, seed=29, ignore_frac=0.0, bias=True)
    g = torch.Generator().manual_seed(8)
    lab[torch.randperm(1100, generator=g)[:650]] = IGNORE
    hd, wd, ld, bd = h.to(gpu, torch.bfloat16), w.to(gpu, torch.bfloat16), lab.to(gpu), b.to(gpu)
    for red in (_lib.CCE_REDUCTION_MEAN, _lib.CCE_REDUCTION_NONE):
        out = {}
        for rows in (_lib.CCE_LSE_ALL_ROWS, _lib.CCE_LSE_LABELLED_ROWS):
            out[rows] = [t.cpu() for t in torch.ops.chronicals_hip.cce_fwd(hd, wd, ld, bd, IGNORE, 0.1, 1e-3, 0,
                                                                             red, rows)]
        (l0, s0, n0, t0), (l1, s1, n1, t1) = out[0], out[1]
        valid = lab != IGNORE
        assert int(n0) == int(n1) == int(valid.sum())
        assert_loss_close(l1.numpy(), l0.numpy(), "loss", rtol=1e-5)
        np.testing.assert_allclose(s1[valid].numpy(), s0[valid].numpy(), rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(t1[valid].numpy(), t0[valid].numpy(), rtol=1e-6, atol=1e-6)
        assert not s1[~valid].any() and not t1[~valid].any()
    # the autograd path runs on the labelled-rows forward: against the oracle
    compare(run_hip(gpu, h, w, lab, b, chunk=1024), run_oracle(h, w, lab, b, chunk=1024), f"lse_rows d={d}")


@pytest.mark.parametrize("N,keep", [
    (65536, 0.5),     # 256 row tiles, 128 live: room for 64 splits per live tile
    (2 ** 20, 0.97),  # 4096 row tiles: the launch is capped at 8192 workgroups, 2 splits per tile
    (2 ** 20, 0.01),  # 4096 row tiles, about 40 live: the capped launch still allows 64 per tile
])
def test_forward_labelled_rows_resplits_vocabulary(gpu, N, keep):
    """Many row tiles, some of them ignored: the compacted forward re-splits
    the vocabulary over its live row tiles on the device, within the
    workgroups its launch holds, and must give the all-rows forward's lse."""
    from chronicals_amd import _lib
    print(f"case resplit N={N} keep={keep}", flush=True)
    d, V = 64, 20000
    g = torch.Generator().manual_seed(31)
    h = (torch.randn(N, d, generator=g)).to(gpu, torch.bfloat16)
    w = (torch.randn(V, d, generator=g) * 0.2).to(gpu, torch.bfloat16)
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) >= keep] = IGNORE
    ld = lab.to(gpu)
    out = {}
    for rows in (_lib.CCE_LSE_ALL_ROWS, _lib.CCE_LSE_LABELLED_ROWS):
        out[rows] = [t.cpu() for t in torch.ops.chronicals_hip.cce_fwd(h, w, ld, None, IGNORE, 0.0, 0.0, 0,
                                                                         _lib.CCE_REDUCTION_MEAN, rows)]
    (l0, s0, n0, _), (l1, s1, n1, _) = out[0], out[1]
    valid = lab != IGNORE
    assert int(n0) == int(n1) == int(valid.sum())
    assert_loss_close(float(l1), float(l0), "loss", rtol=1e-5)
    np.testing.assert_allclose(s1[valid].numpy(), s0[valid].numpy(), rtol=1e-6, atol=1e-6)
    assert not s1[~valid].any()


def test_empty_batch(gpu):
    h = torch.zeros(0, 64)
    w = torch.randn(300, 64) * 0.02
    lab = torch.zeros(0, dtype=torch.int64)
    got = run_hip(gpu, h, w, lab)
    assert float(got["loss"]) == 0.0
    assert got["dw"].shape == (300, 64) and not np.any(got["dw"])


def test_frozen_weight_and_int32_labels_and_3d(gpu):
    h, w, lab, _ = _rand_case(2 * 150, 80, 1500, seed=21)
    h3 = h.reshape(2, 150, 80)
    lab3 = lab.reshape(2, 150).to(torch.int32)
    got = run_hip(gpu, h3, w, lab3, need_dw=False)
    ref = run_oracle(h, w, lab)
    assert got["dw"] is None
    assert_loss_close(got["loss"], ref["loss"])
    assert_grad_close(got["dh"].reshape(ref["dh"].shape), ref["dh"], "dh (frozen W)")


@pytest.mark.parametrize("need_dh,need_dw,need_db", [(True, False, False), (False, True, False),
                                                    (False, False, True), (False, True, True)])
def test_gradient_subsets_banded(gpu, need_dh, need_dw, need_db):
    """Every subset of requested gradients through the banded backward (d % 64 == 0, several
    bands, so the per-band launch alternates its two G buffers)."""
    print(f"case dh={need_dh} dw={need_dw} db={need_db}", flush=True)
    h, w, lab, b = _rand_case(450, 384, 2600, seed=31, bias=True)
    got = run_hip(gpu, h, w, lab, b, chunk=512, need_dh=need_dh, need_dw=need_dw, need_db=need_db)
    ref = run_oracle(h, w, lab, b, chunk=512)
    assert_loss_close(got["loss"], ref["loss"])
    for k, need in (("dh", need_dh), ("dw", need_dw), ("db", need_db)):
        if need:
            assert_grad_close(got[k], ref[k], f"{k} (subset)")
        else:
            assert got[k] is None


def test_fp32_and_fp16_inputs_return_input_dtypes(gpu):
    h, w, lab, _ = _rand_case(128, 64, 900, seed=4)
    from chronicals_amd.kernels.cut_cross_entropy import cut_cross_entropy
    for dt in (torch.float32, torch.float16):
        hd = h.to(gpu, dt).requires_grad_(True)
        wd = w.to(gpu, dt).requires_grad_(True)
        loss = cut_cross_entropy(hd, wd, lab.to(gpu))
        loss.backward()
        assert loss.dtype == torch.float32 and hd.grad.dtype == dt and wd.grad.dtype == dt
        ref = run_oracle(h, w, lab)
        assert_loss_close(loss.item(), ref["loss"])
        assert_grad_close(hd.grad.float().cpu().numpy(), ref["dh"], f"dh {dt}")
        assert_grad_close(wd.grad.float().cpu().numpy(), ref["dw"], f"dw {dt}")


def test_c1_full_vs_oracle(gpu):
    """C1 (N=256, d=768, V=50257, fp32 inputs, 10% ignored) at full size."""
    cfg = CONFIGS["C1"]
    h, w, lab = make_inputs(cfg, seed=0)
    print("case C1 full", flush=True)
    got = run_hip(gpu, h, w, lab, chunk=8192, hdtype=torch.float32, wdtype=torch.float32)
    ref = run_oracle(h, w, lab, chunk=8192)
    compare(got, ref, "C1")
    # against the unrounded fp32 inputs too: the bf16 rounding at the boundary stays inside the contract
    raw = oracle.loss_and_grads(h.numpy(), w.numpy(), lab.numpy(), chunk_size=8192)
    assert_loss_close(got["loss"], raw[0], "C1 loss vs fp32 oracle")
    assert_grad_close(got["dh"], raw[2], "C1 dh vs fp32 oracle")
    assert_grad_close(got["dw"], raw[3], "C1 dw vs fp32 oracle")


@pytest.mark.parametrize("name,n", [("C2", 512), ("C3", 256), ("C4", 512), ("C5", 256)])
def test_config_row_slice_vs_oracle(gpu, name, n):
    """Full d and V of each configuration on a slice of rows (the oracle's cost is linear in N)."""
    cfg = CONFIGS[name]
    print(f"case {name} rows={n}", flush=True)
    h, w, lab = make_inputs(cfg, seed=0, N=n)
    got = run_hip(gpu, h, w, lab)
    ref = run_oracle(h, w, lab)
    compare(got, ref, f"{name}[:{n}]")


def test_deterministic(gpu):
    h, w, lab, b = _rand_case(700, 128, 4000, seed=8, bias=True)
    a = run_hip(gpu, h, w, lab, b, chunk=1024)
    c = run_hip(gpu, h, w, lab, b, chunk=1024)
    for k in ("loss", "dh", "dw", "db"):
        assert np.array_equal(a[k], c[k]), k


def test_side_streams_concurrent_no_host_sync(gpu):
    """The ops launch on the caller's current stream, keep no state between
    calls and never synchronise with the host: two problems, forward and
    backward, are issued on two side streams (default priority) under torch's
    sync debug mode "error" (a synchronising torch call raises), then compared
    bitwise with the same problems run one after the other on the default
    stream.  Each side stream first spins for a bounded time and only then
    makes the input copies the op reads, so a launch on any other stream
    would read them before they are written."""
    cases = [_rand_case(700, 128, 4000, seed=21, bias=True), _rand_case(1300, 256, 9000, seed=22)]
    refs = [run_hip(gpu, h, w, lab, b, chunk=2048) for h, w, lab, b in cases]
    sources = []
    for h, w, lab, b in cases:
        sources.append((h.to(gpu, torch.bfloat16), w.to(gpu, torch.bfloat16), lab.to(gpu),
                        None if b is None else b.to(gpu, torch.float32)))
    main = torch.cuda.current_stream(gpu)
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    prepared, losses = [], []
    torch.cuda.set_sync_debug_mode("error")
    try:
        for s, (h0, w0, l0, b0) in zip(streams, sources):
            s.wait_stream(main)
            with torch.cuda.stream(s):
                torch.cuda._sleep(20_000_000)  # about 10 ms of spinning on this stream
                hd = h0.clone().requires_grad_(True)
                wd = w0.clone().requires_grad_(True)
                bd = None if b0 is None else b0.clone().requires_grad_(True)
                ld = l0.clone()
                loss = _cce()(hd, wd, ld, bd, 2048, IGNORE, 0.0, 0.0)
                loss.backward()
                prepared.append((hd, wd, ld, bd))
                losses.append(loss)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    for i, (ref, (hd, wd, ld, bd), loss) in enumerate(zip(refs, prepared, losses)):
        assert np.array_equal(loss.detach().float().cpu().numpy(), ref["loss"]), f"case {i} loss"
        assert np.array_equal(hd.grad.float().cpu().numpy(), ref["dh"]), f"case {i} dh"
        assert np.array_equal(wd.grad.float().cpu().numpy(), ref["dw"]), f"case {i} dw"
        if bd is not None:
            assert np.array_equal(bd.grad.float().cpu().numpy(), ref["db"]), f"case {i} db"


@pytest.mark.parametrize("name", ["C2", "C3", "C4", "C5"])
def test_full_size_vs_torch_fp32(gpu, name):
    """Every benchmark configuration at full size against an fp32 torch
    reference that materialises the logits (4096 rows at a time) on the GPU,
    from the same bf16-rounded inputs."""
    cfg = CONFIGS[name]
    print(f"case {name} full vs torch fp32", flush=True)
    h, w, lab = make_inputs(cfg, seed=0, device=gpu, gen_device="cuda")
    hd = h.detach().to(torch.bfloat16).requires_grad_(True)
    wd = w.detach().to(torch.bfloat16).requires_grad_(True)
    loss = _cce()(hd, wd, lab, None, 8192, IGNORE, 0.0, 0.0, reduction=cfg.reduction)
    loss.backward()
    torch.cuda.synchronize()
    ref = torch_reference_rows(hd.detach(), wd.detach(), lab, dtype=torch.float32)
    rep = {"dh": grad_report_torch(hd.grad, ref["dh"]), "dw": grad_report_torch(wd.grad, ref["dw"])}
    print(f"{name} loss {float(loss.detach()):.6f} ref {float(ref['loss']):.6f} {rep}", flush=True)
    assert_loss_close(float(loss.detach()), float(ref["loss"]), f"{name} loss")
    assert_grad_close_torch(hd.grad, ref["dh"], f"{name} dh")
    assert_grad_close_torch(wd.grad, ref["dw"], f"{name} dw")


def test_custom_ops_opcheck(gpu):
    """chronicals_hip::cce_fwd / cce_bwd: schema (no input mutation or aliasing) and fake-tensor
    implementations agree with the real kernels."""
    import chronicals_amd.ops  # noqa: F401
    h, w, lab, b = _rand_case(200, 64, 900, seed=41, bias=True)
    hd = h.to(gpu, torch.bfloat16).contiguous()
    wd = w.to(gpu, torch.bfloat16).contiguous()
    ld = lab.to(gpu)
    bd = b.to(gpu, torch.float32)
    checks = ("test_schema", "test_faketensor")
    for red in (0, 1, 2):
        torch.library.opcheck(torch.ops.chronicals_hip.cce_fwd.default, (hd, wd, ld, bd, IGNORE, 0.1, 1e-4, red % 2, red),
                              test_utils=checks)
        torch.library.opcheck(torch.ops.chronicals_hip.cce_fwd.default,
                              (hd, wd, ld, bd, IGNORE, 0.1, 1e-4, red % 2, red, 1), test_utils=checks)
    loss, lse, nv, _ = torch.ops.chronicals_hip.cce_fwd(hd, wd, ld, bd, IGNORE, 0.0, 0.0, 0, 1)
    g = torch.tensor(1.0, device=gpu)
    for need in ((True, True, True), (False, True, False), (True, False, True)):
        torch.library.opcheck(torch.ops.chronicals_hip.cce_bwd.default,
                              (g, hd, wd, ld, lse, nv, bd, IGNORE, 0.0, 0.0, 1, 512, *need, False, True),
                              test_utils=checks)


def test_torch_compile_fullgraph_matches_eager(gpu):
    """The op traces into one graph (torch.compile, fullgraph) and gives the eager results."""
    from chronicals_amd.kernels.cut_cross_entropy import cut_cross_entropy
    h, w, lab, b = _rand_case(300, 128, 2000, seed=43, bias=True)

    def loss_fn(hd, wd, ld, bd):
        return cut_cross_entropy(hd, wd, ld, bd, 512, IGNORE, 0.1, 1e-4)

    def run(fn):
        hd = h.to(gpu, torch.bfloat16).requires_grad_(True)
        wd = w.to(gpu, torch.bfloat16).requires_grad_(True)
        bd = b.to(gpu, torch.float32).requires_grad_(True)
        loss = fn(hd, wd, lab.to(gpu), bd)
        loss.backward()  # the compiled graph's backward runs chronicals_hip::cce_bwd
        torch.cuda.synchronize()
        return loss.detach(), hd.grad, wd.grad, bd.grad

    eager = run(loss_fn)
    compiled = run(torch.compile(loss_fn, backend="aot_eager", fullgraph=True))
    for a, c, name in zip(eager, compiled, ("loss", "dh", "dw", "db")):
        assert torch.equal(a, c), name


def test_peak_memory_below_materialised_logits(gpu):
    """The reference's memory test (tests/test_lora_optimizations.py:297-342): fwd+bwd peak memory of the
    fused loss below 0.8x that of materialised logits + F.cross_entropy, at its shape N=1024, d=256, V=32000."""
    import torch.nn.functional as F
    from chronicals_amd.kernels.cut_cross_entropy import cut_cross_entropy
    g = torch.Generator().manual_seed(3)
    h = torch.randn(1024, 256, generator=g).to(gpu, torch.bfloat16).requires_grad_(True)
    w = (torch.randn(32000, 256, generator=g) * 0.02).to(gpu, torch.bfloat16).requires_grad_(True)
    lab = torch.randint(0, 32000, (1024,), generator=g).to(gpu)

    def peak(fn):
        h.grad = None
        w.grad = None
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        fn().backward()
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - base

    p_cce = peak(lambda: cut_cross_entropy(h, w, lab))
    p_mat = peak(lambda: F.cross_entropy((h @ w.t()).float(), lab))
    assert p_cce < 0.8 * p_mat, (p_cce, p_mat)


@pytest.mark.parametrize("cfg", ["C2", "C5"])
def test_peak_memory_bounded(gpu, cfg):
    """The fwd+bwd holds the gradients, the backward workspace (O(N*d) buffers
    plus a band gradient bounded by its 512 MiB budget: at C5 four row blocks)
    and the forward's, never the N x V logits."""
    from chronicals_amd import _lib
    from chronicals_amd.kernels.cut_cross_entropy import cut_cross_entropy
    N, d, V = {"C2": (16384, 896, 151936), "C5": (65536, 3584, 152064)}[cfg]
    chunk = 8192
    g = torch.Generator(device=gpu).manual_seed(0)
    h = torch.randn(N, d, generator=g, device=gpu).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(V, d, generator=g, device=gpu) * 0.02).to(torch.bfloat16).requires_grad_(True)
    lab = torch.randint(0, V, (N,), generator=g, device=gpu)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    cut_cross_entropy(h, w, lab, chunk_size=chunk).backward()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    grads = N * d * 2 + V * d * 2
    bound = (grads + _lib.backward_workspace_bytes(N, d, V, chunk, True, True)
             + _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS)
             + 64 * 2 ** 20)
    print(f"{cfg} peak extra {peak / 2**20:.0f} MiB, bound {bound / 2**20:.0f} MiB, "
          f"materialised fp32 logits + grad {N * V * 8 / 2**20:.0f} MiB", flush=True)
    assert peak <= bound
    assert peak < 0.1 * N * V * 8
    # what is not O(N*d) (H in row order, the fp32 dH accumulator, the
    # gradients) is the bounded band state
    ws = _lib.backward_workspace_bytes(N, d, V, chunk, True, True)
    assert ws - N * (8 * d + 64) <= 512 * 2 ** 20 + 2 * d * chunk * 2 + chunk * d * 4 + 2 ** 20
    # H^T and the band transposes of W live in the gradient outputs until
    # those are written: at C5 the fwd+bwd peak beside the gradients stays
    # within 1.5 GiB
    assert peak - grads <= {"C2": 640, "C5": 1536}[cfg] * 2 ** 20, (peak - grads) / 2 ** 20


@pytest.mark.parametrize("scale", [30.0, 300.0])
def test_fused_extreme_logit_magnitudes(gpu, scale):
    """Large hidden norms (logits of order +-scale*sqrt(d)): the online log-sum-exp stays finite and exact."""
    g = torch.Generator().manual_seed(82)
    h = torch.randn(300, 128, generator=g) * scale
    w = torch.randn(3001, 128, generator=g) * 0.1
    lab = torch.randint(0, 3001, (300,), generator=g)
    got = run_hip(gpu, h, w, lab, z=1e-6)
    ref = run_oracle(h, w, lab, z=1e-6)
    assert np.isfinite(got["loss"]).all()
    assert_loss_close(got["loss"], ref["loss"], "loss")
    assert_grad_close(got["dh"], ref["dh"], "dh")
    assert_grad_close(got["dw"], ref["dw"], "dw")


@pytest.mark.parametrize("ignore_frac,bias", [(0.0, False), (0.4, True), (1.0, False)])
def test_compute_z_loss(gpu, ignore_frac, bias):
    """compute_z_loss (reference cut_cross_entropy.py:1379-1400) = mean over the
    labelled rows of lse^2, against the oracle's lse; every row ignored gives 0
    (the reference's denominator is clamped to 1)."""
    from chronicals_amd.kernels.cut_cross_entropy import compute_z_loss
    print(f"case compute_z_loss ignore_frac={ignore_frac} bias={bias}", flush=True)
    h, w, lab, b = _rand_case(700, 192, 5001, seed=41, ignore_frac=ignore_frac, bias=bias)
    got = compute_z_loss(h.to(gpu, torch.bfloat16), w.to(gpu, torch.bfloat16), lab.to(gpu),
                         None if b is None else b.to(gpu))
    ref = run_oracle(h, w, lab, b)
    valid = (lab != IGNORE).numpy()
    want = float((ref["lse"][valid] ** 2).sum() / max(valid.sum(), 1))
    assert not got.requires_grad
    if valid.any():
        assert_loss_close(float(got), want, "z-loss")
    else:
        assert float(got) == 0.0


def test_linear_cross_entropy_name(gpu):
    """linear_cross_entropy (the name the reference's trainer imports) takes
    (hidden, weight, labels, bias, ignore_index, reduction) and gives
    cut_cross_entropy's loss and gradients."""
    from chronicals_amd.kernels.cut_cross_entropy import linear_cross_entropy
    h, w, lab, b = _rand_case(300, 128, 3001, seed=43, bias=True)
    hd = h.to(gpu, torch.bfloat16).requires_grad_(True)
    wd = w.to(gpu, torch.bfloat16).requires_grad_(True)
    bd = b.to(gpu).requires_grad_(True)
    loss = linear_cross_entropy(hd, wd, lab.to(gpu), bd, IGNORE, "sum")
    loss.backward()
    got = {"loss": loss.detach().cpu().numpy(), "dh": hd.grad.float().cpu().numpy(),
           "dw": wd.grad.float().cpu().numpy(), "db": bd.grad.float().cpu().numpy()}
    compare(got, run_oracle(h, w, lab, b, reduction="sum"), "linear_cross_entropy")


@pytest.mark.parametrize("N,d,V,chunk,budget_mb,ignore_frac,bias,kw", [
    (1500, 256, 5000, 2048, 0, 0.3, False, {}),   # one block, 6 live row tiles of 6
    (2100, 320, 7000, 1024, 2, 0.1, True, {}),    # row blocks of 512 + bias; 256 + 128-wide dH tiles
    (700, 128, 3000, 1024, 0, 0.97, False, {}),   # 21 labelled rows: one live tile, the rest zero-filled
    # fp32 operands and gradients (in-place accumulation), sum, smoothing and z-loss
    (1200, 192, 6000, 2048, 0, 0.2, True, dict(hdtype=torch.float32, wdtype=torch.float32, reduction="sum",
                                                eps=0.1, z=1e-4)),
    # frozen weight (dH only) in row blocks, per-row grad_output
    (1800, 256, 4000, 1024, 1, 0.1, False, dict(need_dw=False, reduction="none")),
])
def test_row_order_reads_match_gathered_copy(gpu, monkeypatch, N, d, V, chunk, budget_mb, ignore_frac, bias, kw):
    """With CHRONICALS_CCE_ROW_GATHER=1 the compacted GEMMs read H's rows
    through the row order (the default for H of 256 MiB to 2 GiB); with =0
    they read a gathered copy of H (the default below and above).  Same
    values in the same order: loss, dH, dW and dB bitwise equal, and the
    copy's N x d bf16 shows in both workspaces."""
    from chronicals_amd import _lib
    print(f"case row order N={N} d={d} V={V} chunk={chunk} budget={budget_mb} ignore={ignore_frac}", flush=True)
    if budget_mb:
        monkeypatch.setenv("CHRONICALS_CCE_G_BUDGET_MB", str(budget_mb))
    monkeypatch.setenv("CHRONICALS_CCE_ROW_GATHER", "1")
    h, w, lab, b = _rand_case(N, d, V, seed=N + 11, ignore_frac=ignore_frac, bias=bias)
    ws_b = _lib.backward_workspace_bytes(N, d, V, chunk, True, True)
    ws_f = _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS)
    kw = dict(kw)
    go = None
    if kw.get("reduction") == "none":
        go = torch.rand(N, generator=torch.Generator().manual_seed(9))
        kw["grad_output"] = go
    got = run_hip(gpu, h, w, lab, b, chunk=chunk, **kw)
    ref = run_oracle(h, w, lab, b, chunk=chunk, eps=kw.get("eps", 0.0), z=kw.get("z", 0.0),
                     reduction=kw.get("reduction", "mean"), grad_output=go)
    compare(got, ref, f"row order N{N}")
    monkeypatch.setenv("CHRONICALS_CCE_ROW_GATHER", "0")
    assert _lib.backward_workspace_bytes(N, d, V, chunk, True, True) >= ws_b + N * d * 2
    assert _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS) >= ws_f + N * d * 2
    copy = run_hip(gpu, h, w, lab, b, chunk=chunk, **kw)
    for k in ("loss", "dh", "dw", "db"):
        if got[k] is not None:
            assert np.array_equal(got[k], copy[k]), k


@pytest.mark.parametrize("N,d,V,chunk,budget_mb,hdtype,reduction,bias,frozen,ignore_frac", [
    # 6 row blocks of 256 (2048-column bands); dH split 4 ways per block, folded into the next launch
    (1300, 128, 9000, 1024, 2, torch.bfloat16, "mean", False, False, 0.1),
    # fp32 gradients accumulate in place over bands (dH) and blocks (dW); dB added over the blocks
    (2100, 256, 7000, 2048, 4, torch.float32, "sum", True, False, 0.1),
    # d % 64 != 0: the unbanded path in 4 blocks, per-row grad_output
    (1000, 72, 5000, 1024, 1, torch.bfloat16, "none", True, False, 0.1),
    # frozen weight (dH only), 6 blocks of 512
    (3000, 512, 12000, 4096, 8, torch.bfloat16, "mean", False, True, 0.1),
    # 60% of the rows ignored: the blocks past the live rows have no rows to run; 256 + 128-wide dH tiles
    (2600, 320, 8000, 2048, 4, torch.float32, "mean", False, False, 0.6),
    # 3 blocks of 2048 rows x 16 hidden tiles: dH unsplit
    (4500, 4096, 2000, 1024, 8, torch.bfloat16, "mean", True, False, 0.05),
])
def test_row_blocks(gpu, monkeypatch, N, d, V, chunk, budget_mb, hdtype, reduction, bias, frozen, ignore_frac):
    """A backward whose band gradient exceeds the memory budget runs in row
    blocks (CHRONICALS_CCE_G_BUDGET_MB shrinks the budget so small problems
    take several): dW and dB of a band accumulate over the blocks, dH over the
    bands; against the oracle and bitwise repeatable."""
    from chronicals_amd import _lib
    print(f"case row blocks N={N} d={d} V={V} chunk={chunk} budget={budget_mb}MiB {hdtype} {reduction}", flush=True)
    f32 = hdtype == torch.float32
    ws_default = _lib.backward_workspace_bytes(N, d, V, chunk, True, not frozen, f32, f32)
    monkeypatch.setenv("CHRONICALS_CCE_G_BUDGET_MB", str(budget_mb))
    # the budget took effect (the band gradient shrinks; an fp32 dW accumulator may be added)
    assert _lib.backward_workspace_bytes(N, d, V, chunk, True, not frozen, f32, f32) != ws_default
    h, w, lab, b = _rand_case(N, d, V, seed=N + d + 7, ignore_frac=ignore_frac, bias=bias)
    go = torch.rand(N, generator=torch.Generator().manual_seed(5)) if reduction == "none" else None
    kw = dict(chunk=chunk, reduction=reduction, grad_output=go, hdtype=hdtype, wdtype=hdtype, need_dw=not frozen)
    got = run_hip(gpu, h, w, lab, b, **kw)
    compare(got, run_oracle(h, w, lab, b, chunk=chunk, reduction=reduction, grad_output=go), f"blocks N{N}d{d}")
    again = run_hip(gpu, h, w, lab, b, **kw)
    assert np.array_equal(got["dh"], again["dh"])
    if not frozen:
        assert np.array_equal(got["dw"], again["dw"])


@pytest.mark.parametrize("N,d,V,chunk,budget_mb,hdtype,wdtype,need_dw,bias", [
    # 2 bands, 4 row blocks: H^T in grad_hidden; band 0's W^T in band 1's dW
    # rows, band 1's (the last) in its own rows, transposed by a launch of its
    # own after band 0, and its dW written from the fp32 accumulator at the end
    (4096, 64, 500, 256, 1, torch.bfloat16, torch.bfloat16, True, False),
    # fp32 dW (accumulates in place): the last band's W^T in a workspace buffer
    (4096, 64, 500, 256, 1, torch.bfloat16, torch.float32, True, True),
    # fp32 dH (its own accumulator): H^T stays in the workspace
    (4096, 64, 500, 256, 1, torch.float32, torch.bfloat16, True, False),
    # N % 64 != 0: H^T in the workspace; 4 bands in one block, W^T in the next
    # band's dW rows, the last band's in a workspace buffer
    (4100, 64, 900, 256, 0, torch.bfloat16, torch.bfloat16, True, False),
    # 5 bands in 2 blocks, 256 + 128-wide hidden tiles, bias
    (4096, 320, 1200, 256, 2, torch.bfloat16, torch.bfloat16, True, True),
    # frozen weight, N >= 2 x band: both W^T buffers in grad_hidden
    (4096, 128, 900, 256, 0, torch.bfloat16, torch.bfloat16, False, False),
    # frozen weight, N < 2 x band: W^T in the workspace
    (300, 128, 900, 256, 0, torch.bfloat16, torch.bfloat16, False, False),
])
def test_gradient_outputs_as_scratch(gpu, monkeypatch, N, d, V, chunk, budget_mb, hdtype, wdtype, need_dw, bias):
    """While the bands run, H^T and the band transposes of W live in gradient
    output memory that is not yet written (grad_hidden; the rows of the next
    band of grad_weight); each placement and its fallback against the oracle,
    and bitwise repeatable."""
    print(f"case outputs-as-scratch N={N} d={d} V={V} chunk={chunk} budget={budget_mb} {hdtype} {wdtype} "
          f"dw={need_dw} bias={bias}", flush=True)
    if budget_mb:
        monkeypatch.setenv("CHRONICALS_CCE_G_BUDGET_MB", str(budget_mb))
    h, w, lab, b = _rand_case(N, d, V, seed=N + d + V, ignore_frac=0.2, bias=bias)
    kw = dict(chunk=chunk, hdtype=hdtype, wdtype=wdtype, need_dw=need_dw, z=1e-4)
    got = run_hip(gpu, h, w, lab, b, **kw)
    ref = run_oracle(h, w, lab, b, chunk=chunk, z=1e-4)
    if not need_dw:
        ref["dw"] = None
    compare(got, ref, f"scratch N{N}d{d}V{V}")
    again = run_hip(gpu, h, w, lab, b, **kw)
    assert np.array_equal(got["dh"], again["dh"])
    if need_dw:
        assert np.array_equal(got["dw"], again["dw"])


def _sweep_cases(n=40, seed=2026):
    """Seeded random problems that mix every layout switch of the fused path:
    ragged N / d / V, band width, row blocks (G budget), row-order reads or
    the gathered copy, split dH, ignored rows, bias, dtypes, reductions,
    smoothing forms and z-loss."""
    import random
    rng = random.Random(seed)
    out = []
    for i in range(n):
        d = rng.choice([8, 64, 72, 128, 192, 256, 320, 384, 448, 640])
        N = rng.choice([1, 17, 255, 256, 257, 700, 1100, 1600, 2400, 3000])
        V = rng.choice([7, 300, 1000, 2049, 5003, 9000, 15000])
        out.append(dict(
            N=N, d=d, V=V, seed=1000 + i,
            chunk=rng.choice([256, 512, 1024, 2048, 8192]),
            budget=rng.choice([0, 0, 1, 2, 4]),
            gather=rng.choice(["", "0", "1"]),
            ignore=rng.choice([0.0, 0.1, 0.5, 0.95]),
            bias=rng.random() < 0.4,
            dtype=rng.choice([torch.bfloat16, torch.bfloat16, torch.float32, torch.float16]),
            reduction=rng.choice(["mean", "mean", "sum", "none"]),
            eps=rng.choice([0.0, 0.0, 0.1]),
            z=rng.choice([0.0, 1e-4]),
            need_dw=rng.random() < 0.8))
    return out


# CHRONICALS_SWEEP_CASES widens the sweep for a one-off extended run (default 40)
@pytest.mark.parametrize("case", _sweep_cases(int(os.environ.get("CHRONICALS_SWEEP_CASES", "40"))),
                         ids=lambda c: f"N{c['N']}d{c['d']}V{c['V']}s{c['seed']}")
def test_random_sweep(gpu, monkeypatch, case):
    """Seeded random problems against the oracle (loss and every gradient)."""
    c = case
    print(f"case sweep {c}", flush=True)
    if c["budget"]:
        monkeypatch.setenv("CHRONICALS_CCE_G_BUDGET_MB", str(c["budget"]))
    if c["gather"]:
        monkeypatch.setenv("CHRONICALS_CCE_ROW_GATHER", c["gather"])
    h, w, lab, b = _rand_case(c["N"], c["d"], c["V"], seed=c["seed"], ignore_frac=c["ignore"], bias=c["bias"])
    go = None
    if c["reduction"] == "none":
        go = torch.rand(c["N"], generator=torch.Generator().manual_seed(c["seed"]))
    got = run_hip(gpu, h, w, lab, b, chunk=c["chunk"], eps=c["eps"], z=c["z"], reduction=c["reduction"],
                  grad_output=go, need_dw=c["need_dw"], hdtype=c["dtype"], wdtype=c["dtype"])
    # the boundary rounds the operands it is given to bf16: fp16 operands are
    # first rounded to fp16 (a double rounding the oracle must see too)
    ho, wo = (h.to(torch.float16).float(), w.to(torch.float16).float()) if c["dtype"] == torch.float16 else (h, w)
    ref = run_oracle(ho, wo, lab, b, chunk=c["chunk"], eps=c["eps"], z=c["z"], reduction=c["reduction"],
                     grad_output=go)
    if not c["need_dw"]:
        ref["dw"] = None
    compare(got, ref, f"sweep {c['seed']}")


@pytest.mark.parametrize("N,d,V,chunk,where", [
    # H^T in grad_hidden (bf16 dH, several bands, N % 64 == 0): past it lies
    # whatever follows the caller's buffer
    (1088, 128, 3000, 1024, "grad_hidden"),  # N % 64 == 0, N % 256 != 0: H^T in grad_hidden
    (1000, 128, 3000, 1024, "workspace"),    # N % 64 != 0: H^T padded to 1024 columns in the workspace
    (1000, 320, 3000, 1024, "workspace"),    # 256 + 128-wide hidden tiles
    # H^T in the workspace (N % 64 != 0, or one band, or fp32 dH): past it
    # lies the rest of the workspace
    (1001, 128, 3000, 1024, "workspace"),
    (1000, 128, 1000, 1024, "workspace"),
    (999, 72, 2000, 512, "workspace"),       # d % 64 != 0: the separate dW launch
])
def test_dw_reads_stop_at_the_end_of_ht(gpu, N, d, V, chunk, where):
    """dW = G^T . H reads H^T ([d][N rounded up to 8]) in 64-row slabs of N;
    when N is not a multiple of 64 the last slab runs past the end of H^T's
    last row.  Those reads must come back as zeros: with the memory just past
    H^T holding NaN (the tail of a larger buffer that holds grad_hidden, or a
    NaN-filled workspace), dW stays finite and matches the oracle."""
    print(f"case ht-end N={N} d={d} V={V} chunk={chunk} {where}", flush=True)
    from chronicals_amd import _lib
    from chronicals_amd.ops import _stream
    lib = _lib.load()
    h, w, lab, _ = _rand_case(N, d, V, seed=N + d, ignore_frac=0.0)
    hd = h.to(gpu, torch.bfloat16).contiguous()
    wd = w.to(gpu, torch.bfloat16).contiguous()
    ld = lab.to(gpu)
    loss, lse, n_valid, _ = torch.ops.chronicals_hip.cce_fwd(hd, wd, ld, None, IGNORE, 0.0, 0.0, 0,
                                                             _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS)
    nan16 = torch.tensor(0x7fc0, dtype=torch.int16).view(torch.bfloat16).item()
    # grad_hidden at the start of a larger NaN-filled buffer
    dh_buf = torch.full((N * d + 8192,), nan16, dtype=torch.bfloat16, device=gpu)
    dh = dh_buf[:N * d]
    dw = torch.empty((V, d), dtype=torch.bfloat16, device=gpu)
    ws = torch.full((_lib.backward_workspace_bytes(N, d, V, chunk, True, True),), 0xFF, dtype=torch.uint8,
                    device=gpu)
    go = torch.ones(1, dtype=torch.float32, device=gpu)
    _lib.check(lib.cce_backward(
        go.data_ptr(), hd.data_ptr(), wd.data_ptr(), ld.data_ptr(), 1, None, lse.data_ptr(), n_valid.data_ptr(),
        N, d, V, IGNORE, 0.0, 0.0, _lib.CCE_REDUCTION_MEAN, chunk,
        dh.data_ptr(), _lib.CCE_DTYPE_BF16, dw.data_ptr(), _lib.CCE_DTYPE_BF16, None,
        ws.data_ptr(), ws.numel(), _stream(gpu)))
    torch.cuda.synchronize()
    got_dw = dw.float().cpu().numpy()
    got_dh = dh.float().cpu().numpy().reshape(N, d)
    assert np.isfinite(got_dw).all(), f"non-finite dW columns: {np.where(~np.isfinite(got_dw).all(0))[0]}"
    assert np.isfinite(got_dh).all()
    ref = run_oracle(h, w, lab, chunk=chunk)
    assert_grad_close(got_dw, ref["dw"], "dW")
    assert_grad_close(got_dh, ref["dh"], "dH")


@pytest.mark.parametrize("name", ["C2", "C5"])
def test_full_size_properties(gpu, name):
    """Size-independent properties at a configuration's full size.

    Linearity: the backward scales G by grad_output/n_valid, so grad_output = 2
    gives exactly twice both gradients (a power of two commutes with every
    rounding step: the exp2 argument does not depend on it, and the bf16
    conversions, MFMA sums and fp32 accumulators scale exactly), bitwise.

    dW's column sums vanish: with no smoothing and no z-loss each labelled row
    of G sums to zero over the vocabulary (softmax minus one-hot), so
    sum_v dW[v, c] = sum_n H[n, c] * sum_v G[n, v] = 0.  What remains is
    rounding: each G element is rounded to bf16 after an fp32 exp2 (relative
    error below 2^-8) and sum_v |G[n, v]| <= 2 * scale, so the row sums are off
    by at most 2^-7 * scale; each dW element is rounded to bf16 once more
    (2^-9 relative).  Per column: |sum_v dW| <= 2^-7 * scale * sum_n |H[n, c]|
    + 2^-9 * sum_v |dW[v, c]|, scale = 1 / n_valid."""
    cfg = CONFIGS[name]
    print(f"case {name} full-size properties", flush=True)
    h, w, lab = make_inputs(cfg, seed=3, device=gpu, gen_device="cuda")
    grads = []
    for go in (1.0, 2.0):
        hd = h.detach().to(torch.bfloat16).requires_grad_(True)
        wd = w.detach().to(torch.bfloat16).requires_grad_(True)
        loss = _cce()(hd, wd, lab, None, 8192, IGNORE, 0.0, 0.0, reduction=cfg.reduction)
        loss.backward(torch.tensor(go, device=gpu))
        torch.cuda.synchronize()
        grads.append((hd.grad.detach(), wd.grad.detach()))
        del hd, wd, loss
    (dh1, dw1), (dh2, dw2) = grads
    assert torch.equal(dh2, dh1 * 2), "dH is not exactly linear in grad_output"
    assert torch.equal(dw2, dw1 * 2), "dW is not exactly linear in grad_output"
    n_valid = int((lab != IGNORE).sum())
    scale = (1.0 / n_valid) if cfg.reduction == "mean" else 1.0
    colsum = dw1.double().sum(0).abs()
    bound = 2.0 ** -7 * scale * h.double().abs().sum(0) + 2.0 ** -9 * dw1.double().abs().sum(0)
    ratio = float((colsum / bound).max())
    # a gradient that loses the one-hot term (the reference CPU path's bug)
    # has row sums of exactly `scale`, so its column sums are
    # scale * sum_n H[n] over the labelled rows; with the term, the
    # random-signed row-sum rounding leaves about 2^-8 of that in norm
    lab_rows = (lab != IGNORE)
    planted = scale * h.double()[lab_rows].sum(0)
    rel = float(dw1.double().sum(0).norm() / planted.norm())
    print(f"{name} max |sum_v dW| / bound = {ratio:.3e}; |sum_v dW| / |without one-hot| = {rel:.3e}", flush=True)
    assert ratio <= 1.0, ratio
    assert rel <= 0.05, rel
    del grads, dh1, dw1, dh2, dw2
    torch.cuda.empty_cache()
