"""Golden fixtures (tests/golden/cce_golden.npz, float64 closed form) against the oracle and the HIP path."""
import os

import numpy as np
import pytest

from oracle import cce_oracle as oracle
from tests.cce_common import IGNORE, assert_grad_close, assert_loss_close

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cce_golden.npz")


def cases():
    z = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in z.files})
    for n in names:
        yield n, {k.split("/")[1]: z[k] for k in z.files if k.startswith(n + "/")}


CASES = list(cases())


@pytest.mark.parametrize("name,c", CASES, ids=[n for n, _ in CASES])
def test_oracle_matches_golden(name, c):
    eps, zw = c["params"]
    red = str(c["reduction"])
    bias = c["bias"] if c["bias"].size else None
    go = c["grad_output"]
    loss, lse, gh, gw, gb = oracle.loss_and_grads(c["hidden"], c["weight"], c["labels"], bias, chunk_size=128,
                                                  label_smoothing=eps, z_loss_weight=zw, reduction=red,
                                                  grad_output=go)
    np.testing.assert_allclose(loss, c["loss"], rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(lse, c["lse"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gh, c["dh"], rtol=2e-4, atol=2e-6)
    np.testing.assert_allclose(gw, c["dw"], rtol=2e-4, atol=2e-6)
    if bias is not None:
        np.testing.assert_allclose(gb, c["db"], rtol=2e-4, atol=2e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("name,c", CASES, ids=[n for n, _ in CASES])
def test_hip_matches_golden(gpu, name, c):
    import torch

    from chronicals_amd.kernels.cut_cross_entropy import cut_cross_entropy

    eps, zw = c["params"]
    red = str(c["reduction"])
    h = torch.from_numpy(c["hidden"]).to(gpu, torch.bfloat16).requires_grad_(True)
    w = torch.from_numpy(c["weight"]).to(gpu, torch.bfloat16).requires_grad_(True)
    lab = torch.from_numpy(c["labels"]).to(gpu)
    b = None
    if c["bias"].size:
        b = torch.from_numpy(c["bias"]).to(gpu, torch.float32).requires_grad_(True)
    loss = cut_cross_entropy(h, w, lab, b, 256, IGNORE, float(eps), float(zw), reduction=red)
    if red == "none":
        loss.backward(torch.from_numpy(c["grad_output"]).to(gpu, torch.float32))
    else:
        loss.backward(torch.tensor(float(c["grad_output"][0]), device=gpu))
    torch.cuda.synchronize()
    assert_loss_close(loss.detach().cpu().numpy(), c["loss"], f"{name} loss")
    assert_grad_close(h.grad.float().cpu().numpy(), c["dh"], f"{name} dh")
    assert_grad_close(w.grad.float().cpu().numpy(), c["dw"], f"{name} dw")
    if b is not None:
        assert_grad_close(b.grad.float().cpu().numpy(), c["db"], f"{name} db")
