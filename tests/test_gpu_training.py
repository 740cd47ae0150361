"""GPU tests of the two callers either side of the path.

Trainer wiring: the HIP loss called the way ChronicalsTrainer's CCE branch
calls it (reference chronicals_trainer.py:1747-1790, set-up :575-594):
hidden states from the model under bf16 autocast, the lm_head weight passed
directly (tied to the embedding, or frozen as under LoRA), label smoothing,
the z-loss default 1e-4 (config.py:283), chunk from get_optimal_chunk_size,
and the loss divided by the gradient-accumulation steps before backward.
Every parameter gradient is compared with the same model trained through a
materialised fp32-logits reference of the loss.

Packed sequences: labels built by the packer's rules
(FixedShapeSequencePacker._create_batch_from_bin, sequence_packer.py:771-842:
-100 padding, first token of every packed sequence after the first masked,
loss_mask = labels != -100), through the fused path and through
compute_padding_free_loss / compute_packed_loss (sequence_packer.py:1660-1717,
sequence_packer_v2.py:1058-1113), against float64 torch on the CPU.

Tolerances: loss within 1e-3 relative; gradients with max abs error
<= 2e-2 * max|ref| and cosine >= 0.9999.
"""
import copy
import math

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import cce_oracle as oracle
from tests.cce_common import IGNORE, assert_grad_close, assert_loss_close, bf16_exact

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


class TinyLM(nn.Module):
    """Embedding -> linear -> tanh -> LayerNorm -> lm_head, HF-like attribute names."""

    def __init__(self, V, d, tied=True, seed=0):
        super().__init__()
        torch.manual_seed(seed)
        self.embed = nn.Embedding(V, d)
        self.proj = nn.Linear(d, d)
        self.norm = nn.LayerNorm(d)
        self.lm_head = nn.Linear(d, V, bias=False)
        nn.init.normal_(self.embed.weight, std=0.02)
        if tied:
            self.lm_head.weight = self.embed.weight
        else:
            nn.init.normal_(self.lm_head.weight, std=0.02)

    def hidden_states(self, ids):
        return self.norm(torch.tanh(self.proj(self.embed(ids))))


def reference_loss(hidden, weight, labels, eps, z):
    """The reference CCE loss on materialised fp32 logits; the value of
    (1-eps)*CE + eps*log(V) + z*lse^2 (cut_cross_entropy.py:674-683) and, for
    autograd, the objective whose logit gradient is the reference backward's
    P - (1-eps)*onehot - eps/V + 2z*lse*P (:767-789)."""
    logits = hidden.float().reshape(-1, hidden.shape[-1]) @ weight.float().t()
    lab = labels.reshape(-1)
    V = logits.shape[-1]
    valid = lab != IGNORE
    lse = torch.logsumexp(logits, dim=-1)
    t = logits.gather(1, torch.where(valid, lab, 0)[:, None])[:, 0]
    ce = (lse - t) * valid
    nv = valid.sum().clamp(min=1)
    value = (((1 - eps) * ce + eps * math.log(V) + z * lse * lse) * valid).sum() / nv
    obj = (((1 - eps) * ce + eps * (lse - logits.mean(dim=-1)) + z * lse * lse) * valid).sum() / nv
    return value, obj


def _trainer_step(model, ids, labels, loss_fn, accum):
    with torch.autocast("cuda", dtype=torch.bfloat16):
        hidden = model.hidden_states(ids)
        loss = loss_fn(hidden, model.lm_head.weight, labels)
    (loss / accum).backward()
    return loss


@pytest.mark.parametrize("tied,frozen_head", [(True, False), (False, False), (False, True)])
def test_trainer_cce_branch_gradients(tied, frozen_head):
    from chronicals_amd.kernels.cut_cross_entropy import CutCrossEntropyLoss, get_optimal_chunk_size

    V, d, B, S, accum, eps, z = 32000, 256, 2, 300, 4, 0.1, 1e-4
    model = TinyLM(V, d, tied=tied).to(DEV)
    if frozen_head:
        model.lm_head.weight.requires_grad_(False)
    ref_model = copy.deepcopy(model)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, V, (B, S), generator=g).to(DEV)
    labels = torch.randint(0, V, (B, S), generator=g)
    labels[:, :5] = IGNORE
    labels = labels.to(DEV)
    print(f"trainer pattern tied={tied} frozen_head={frozen_head}", flush=True)

    chunk = get_optimal_chunk_size(vocab_size=V, hidden_dim=d, available_vram_gb=40.0)
    loss_fn = CutCrossEntropyLoss(chunk_size=chunk, ignore_index=-100, label_smoothing=eps, z_loss_weight=z,
                                  reduction="mean")
    loss = _trainer_step(model, ids, labels, lambda h, w, l: loss_fn(h, w, l, None), accum)

    def ref_fn(h, w, l):
        value, obj = reference_loss(h, w, l, eps, z)
        ref_fn.value = value.detach()
        return obj

    _trainer_step(ref_model, ids, labels, ref_fn, accum)
    torch.cuda.synchronize()
    assert_loss_close(float(loss.detach()), float(ref_fn.value), "loss")
    for (name, p), (_, rp) in zip(model.named_parameters(), ref_model.named_parameters()):
        if not p.requires_grad:
            assert p.grad is None and rp.grad is None, name
            continue
        assert p.grad is not None and p.grad.dtype == p.dtype, name
        assert_grad_close(p.grad.float().cpu().numpy(), rp.grad.float().cpu().numpy(), name)


def pack_labels(seq_labels, max_len, mask_first_token=True):
    """Labels and loss_mask of one packed row, by the packer's rules (sequence_packer.py:771-842)."""
    labels = torch.full((max_len,), IGNORE, dtype=torch.long)
    pos = 0
    for i, sl in enumerate(seq_labels):
        labels[pos:pos + len(sl)] = sl
        if mask_first_token and i > 0:
            labels[pos] = IGNORE
        pos += len(sl)
    return labels, (labels != IGNORE).float()


def _packed_batch(V, rows=2, max_len=1024, seed=0):
    g = torch.Generator().manual_seed(seed)
    labs, masks = [], []
    for _ in range(rows):
        seqs, total = [], 0
        while True:
            n = int(torch.randint(16, 300, (1,), generator=g))
            if total + n > max_len - 40:
                break
            seqs.append(torch.randint(0, V, (n,), generator=g))
            total += n
        lab, m = pack_labels(seqs, max_len)
        labs.append(lab)
        masks.append(m)
    return torch.stack(labs), torch.stack(masks)


def torch_packed_reference(logits, labels, loss_mask, reduction, eps):
    """float64 CPU torch: per-token cross_entropy (label-smoothed), masked, reduced."""
    x = logits.detach().cpu().double().reshape(-1, logits.shape[-1]).requires_grad_(True)
    lab = labels.cpu().reshape(-1)
    loss = F.cross_entropy(x, lab, ignore_index=IGNORE, reduction="none", label_smoothing=eps)
    if loss_mask is not None:
        m = loss_mask.cpu().double().reshape(-1)
        loss = loss * m
        den = m.sum().clamp(min=1.0)
    else:
        den = (lab != IGNORE).sum().clamp(min=1)
    out = loss.sum() / den if reduction == "mean" else (loss.sum() if reduction == "sum" else loss)
    (gx,) = torch.autograd.grad(out, x, torch.ones_like(out))
    return out.detach().numpy(), gx.numpy()


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("eps", [0.0, 0.1])
@pytest.mark.parametrize("with_mask", [True, False])
def test_padding_free_loss_matches_torch(reduction, eps, with_mask):
    from chronicals_amd.kernels.logits_cross_entropy import compute_packed_loss, compute_padding_free_loss

    V = 32000
    labels, mask = _packed_batch(V)
    g = torch.Generator().manual_seed(2)
    logits = (torch.randn(*labels.shape, V, generator=g) * 2).to(torch.bfloat16)
    rl, rg = torch_packed_reference(logits, labels, mask if with_mask else None, reduction, eps)
    print(f"padding-free reduction={reduction} eps={eps} mask={with_mask}", flush=True)
    for fn in (compute_padding_free_loss, compute_packed_loss):
        x = logits.to(DEV).requires_grad_(True)
        loss = fn(x, labels.to(DEV), mask.to(DEV) if with_mask else None, IGNORE, reduction, eps)
        loss.backward(torch.ones_like(loss))
        torch.cuda.synchronize()
        assert_loss_close(loss.detach().cpu().numpy(), rl, "loss")
        assert_grad_close(x.grad.float().cpu().numpy().reshape(rg.shape), rg, "dlogits")


def test_loss_mask_equals_ignore_index_and_weighted_mask():
    from chronicals_amd.kernels.logits_cross_entropy import compute_padding_free_loss

    V = 5000
    labels, mask = _packed_batch(V, rows=3, max_len=512, seed=4)
    g = torch.Generator().manual_seed(5)
    logits = (torch.randn(*labels.shape, V, generator=g) * 2).to(DEV, torch.bfloat16)
    lab = labels.to(DEV)
    a = compute_padding_free_loss(logits, lab, mask.to(DEV))
    b = compute_padding_free_loss(logits, lab)
    assert_loss_close(float(a), float(b), "mask vs ignore_index", rtol=1e-6)
    # a non-binary mask weights tokens
    w = torch.rand(labels.shape, generator=g) * mask
    rl, rg = torch_packed_reference(logits, labels, w, "mean", 0.0)
    x = logits.detach().requires_grad_(True)
    loss = compute_padding_free_loss(x, lab, w.to(DEV))
    loss.backward()
    assert_loss_close(float(loss.detach()), float(rl), "weighted mask")
    assert_grad_close(x.grad.float().cpu().numpy().reshape(rg.shape), rg, "weighted mask dlogits")


def test_fused_path_on_packed_labels_matches_oracle_and_logits_path():
    from chronicals_amd.kernels.cut_cross_entropy import cut_cross_entropy
    from chronicals_amd.kernels.logits_cross_entropy import compute_padding_free_loss

    V, d = 32000, 512
    labels, mask = _packed_batch(V, rows=2, max_len=1024, seed=6)
    g = torch.Generator().manual_seed(7)
    h = torch.randn(*labels.shape, d, generator=g)
    w = torch.randn(V, d, generator=g) * 0.02
    hd = h.to(DEV, torch.bfloat16).requires_grad_(True)
    wd = w.to(DEV, torch.bfloat16).requires_grad_(True)
    loss = cut_cross_entropy(hd, wd, labels.to(DEV))
    loss.backward()
    ol, _, gh, gw, _ = oracle.loss_and_grads(bf16_exact(h).numpy().reshape(-1, d), bf16_exact(w).numpy(),
                                             labels.numpy().reshape(-1))
    torch.cuda.synchronize()
    assert_loss_close(float(loss.detach()), float(ol), "fused loss")
    assert_grad_close(hd.grad.float().cpu().numpy().reshape(gh.shape), gh, "dH")
    assert_grad_close(wd.grad.float().cpu().numpy(), gw, "dW")
    # the same loss through materialised logits and the packed-loss API (eps = 0: both smoothing forms agree)
    logits = (hd.detach().float() @ wd.detach().float().t())
    pl = compute_padding_free_loss(logits, labels.to(DEV), mask.to(DEV))
    assert_loss_close(float(pl), float(loss.detach()), "padding-free vs fused", rtol=1e-4)
    nv = int((labels != IGNORE).sum())
    assert nv == int(mask.sum())
