"""Write tests/golden/cce_golden.npz: small fused linear-CE cases with expected outputs.

Expected values (stored as float32) come from the float64 materialised-logits closed form
(tests/cce_common.torch_reference: torch logsumexp / cross_entropy with
autograd), which is independent of the oracle.  Inputs are rounded to bf16
values (stored as float32) so the HIP path consumes them exactly.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.cce_common import IGNORE, torch_reference  # noqa: E402

CASES = [
    # name, N, d, V, reduction, bias, eps, z, ignore_frac, out_of_range_labels, seed
    ("mean_ignore", 64, 32, 1000, "mean", False, 0.0, 0.0, 0.1, False, 1),
    ("sum_bias_smooth_z", 48, 40, 777, "sum", True, 0.1, 1e-3, 0.05, False, 2),
    ("none_oob", 33, 16, 300, "none", False, 0.0, 0.0, 0.2, True, 3),
    ("mean_all_features", 130, 72, 1031, "mean", True, 0.05, 1e-4, 0.1, True, 4),
]


def bf16_round(x):
    return x.to(torch.bfloat16).to(torch.float32)


def main():
    out = {}
    for name, N, d, V, red, has_bias, eps, z, ign, oob, seed in CASES:
        g = torch.Generator().manual_seed(seed)
        h = bf16_round(torch.randn(N, d, generator=g))
        w = bf16_round(torch.randn(V, d, generator=g) * 0.1)
        lab = torch.randint(0, V, (N,), generator=g)
        lab[torch.rand(N, generator=g) < ign] = IGNORE
        if oob:
            lab[0] = V + 3
            lab[1] = -5
        b = (torch.randn(V, generator=g) * 0.2) if has_bias else None
        go = torch.rand(N, generator=g, dtype=torch.float64) if red == "none" else 0.75
        ref = torch_reference(h, w, lab, b, IGNORE, eps, z, red, dtype=torch.float64,
                              grad_output=go if red == "none" else torch.tensor(go))
        p = name + "/"
        out[p + "hidden"] = h.numpy()
        out[p + "weight"] = w.numpy()
        out[p + "labels"] = lab.numpy()
        out[p + "bias"] = b.numpy() if b is not None else np.zeros(0, np.float32)
        out[p + "params"] = np.array([eps, z], np.float64)
        out[p + "reduction"] = np.array(red)
        out[p + "grad_output"] = np.asarray(go.numpy() if torch.is_tensor(go) else [go], np.float64)
        out[p + "loss"] = ref["loss"].numpy().astype(np.float32)
        out[p + "lse"] = ref["lse"].numpy().astype(np.float32)
        out[p + "dh"] = ref["dh"].numpy().astype(np.float32)
        out[p + "dw"] = ref["dw"].numpy().astype(np.float32)
        out[p + "db"] = ref["db"].numpy().astype(np.float32) if b is not None else np.zeros(0, np.float32)
    path = os.path.join(HERE, "cce_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
