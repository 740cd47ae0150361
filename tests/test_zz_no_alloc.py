"""cce_forward_noalloc: cce_forward with its scratch in the library's static
device array instead of a caller workspace.  Called through the C ABI and
checked against cce_forward on the same inputs (the same kernels run, so the
results must be bitwise equal), on two calls in a row, the second smaller,
and on a case that reuses the array after a larger one left data in it."""
import ctypes

import pytest
import torch

from chronicals_amd import _lib

IGNORE = -100


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _inputs(dev, N, d, V, seed, bias):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(N, d, generator=g).to(dev, torch.bfloat16)
    w = (torch.randn(V, d, generator=g) * 0.05).to(dev, torch.bfloat16)
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < 0.2] = IGNORE
    b = (torch.randn(V, generator=g) * 0.1).to(dev) if bias else None
    return h, w, lab.to(dev), b


def _outputs(dev, N, red):
    loss = torch.full((N if red == _lib.CCE_REDUCTION_NONE else 1,), float("nan"), device=dev)
    lse = torch.full((N,), float("nan"), device=dev)
    tgt = torch.full((N,), float("nan"), device=dev)
    nv = torch.full((1,), -1, dtype=torch.int32, device=dev)
    return loss, lse, tgt, nv


def _run(noalloc, dev, h, w, lab, b, eps, z, form, red, rows):
    lib = _lib.load()
    N, d = h.shape
    V = w.shape[0]
    loss, lse, tgt, nv = _outputs(dev, N, red)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    common = (_ptr(h), _ptr(w), _ptr(lab), 1, _ptr(b), N, d, V, IGNORE, eps, z, form, red, rows,
              _ptr(loss), _ptr(lse), _ptr(tgt), _ptr(nv))
    if noalloc:
        _lib.check(lib.cce_forward_noalloc(*common, stream))
    else:
        nbytes = _lib.forward_workspace_bytes(N, d, V, red, rows)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        _lib.check(lib.cce_forward(*common, _ptr(ws), nbytes, stream))
    torch.cuda.synchronize()
    return [t.cpu() for t in (loss, lse, tgt, nv)]


CASES = [
    # N, d, V, seed, bias, eps, z, smoothing form, reduction, lse rows
    (3000, 256, 20000, 1, True, 0.1, 1e-4, _lib.CCE_SMOOTH_UNIFORM, _lib.CCE_REDUCTION_MEAN,
     _lib.CCE_LSE_LABELLED_ROWS),
    (700, 128, 5003, 2, False, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV, _lib.CCE_REDUCTION_NONE, _lib.CCE_LSE_ALL_ROWS),
    (300, 72, 1000, 3, True, 0.05, 1e-3, _lib.CCE_SMOOTH_LOGV, _lib.CCE_REDUCTION_SUM, _lib.CCE_LSE_LABELLED_ROWS),
]


@pytest.mark.gpu
def test_noalloc_forward_matches_workspace_forward(gpu):
    for case in CASES:  # two or more calls in a row, each smaller than the one before
        N, d, V, seed, bias, eps, z, form, red, rows = case
        print(f"case noalloc N={N} d={d} V={V} red={red} rows={rows}", flush=True)
        h, w, lab, b = _inputs(gpu, N, d, V, seed, bias)
        got = _run(True, gpu, h, w, lab, b, eps, z, form, red, rows)
        want = _run(False, gpu, h, w, lab, b, eps, z, form, red, rows)
        for name, g, e in zip(("loss", "lse", "target", "n_valid"), got, want):
            assert torch.equal(g, e), f"{name} differs for {case}"
        assert int(got[3]) == int((lab != IGNORE).sum())


@pytest.mark.gpu
def test_noalloc_forward_twice_second_smaller(gpu):
    big = (2500, 512, 30000, 5, False, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV, _lib.CCE_REDUCTION_MEAN,
           _lib.CCE_LSE_LABELLED_ROWS)
    small = (400, 512, 30000, 6, False, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV, _lib.CCE_REDUCTION_MEAN,
             _lib.CCE_LSE_LABELLED_ROWS)
    for case in (big, small):
        N, d, V, seed, bias, eps, z, form, red, rows = case
        print(f"case noalloc repeat N={N} d={d} V={V}", flush=True)
        h, w, lab, b = _inputs(gpu, N, d, V, seed, bias)
        got = _run(True, gpu, h, w, lab, b, eps, z, form, red, rows)
        want = _run(False, gpu, h, w, lab, b, eps, z, form, red, rows)
        for name, g, e in zip(("loss", "lse", "target", "n_valid"), got, want):
            assert torch.equal(g, e), f"{name} differs for N={N}"


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", ["C2", "C4"])
def test_noalloc_forward_full_size(gpu, cfg):
    """At full benchmark sizes the labelled-rows forward without a workspace
    reads the hidden rows in place (no N x d copy in the 64 MiB scratch),
    where cce_forward with a workspace gathers them first (H below 256 MiB):
    the same values in the same order, so bitwise equal."""
    N, d, V = {"C2": (16384, 896, 151936), "C4": (32768, 2048, 151936)}[cfg]
    rows = _lib.CCE_LSE_LABELLED_ROWS
    # the workspace forward needs more than the scratch at C4; without a workspace it fits
    if cfg == "C4":
        assert _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, rows) > _lib.CCE_NOALLOC_SCRATCH_BYTES
    print(f"case noalloc full size {cfg}", flush=True)
    h, w, lab, b = _inputs(gpu, N, d, V, 7, False)
    got = _run(True, gpu, h, w, lab, b, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV, _lib.CCE_REDUCTION_MEAN, rows)
    want = _run(False, gpu, h, w, lab, b, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV, _lib.CCE_REDUCTION_MEAN, rows)
    for name, g, e in zip(("loss", "lse", "target", "n_valid"), got, want):
        assert torch.equal(g, e), f"{name} differs at {cfg}"


def test_noalloc_forward_rejects_oversize_problem():
    # the size check comes before any device work: no GPU needed
    lib = _lib.load()
    N, d, V = 2 ** 21, 1024, 152064
    need = _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS)
    assert need > _lib.CCE_NOALLOC_SCRATCH_BYTES
    z = ctypes.c_void_p(0)
    rc = lib.cce_forward_noalloc(z, z, z, 1, z, N, d, V, IGNORE, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV,
                                 _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS, z, z, z, z, z)
    assert rc == _lib.CCE_ERR_WORKSPACE
    assert "static scratch" in lib.cce_last_error().decode()
