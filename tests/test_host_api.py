"""Host-side API of chronicals_amd.kernels.cut_cross_entropy (no GPU needed).

Mirrors the reference module's helpers (chronicals/kernels/cut_cross_entropy.py):
get_optimal_chunk_size :59-90, estimate_memory_savings :1403-1430,
CutCrossEntropyLoss :1081-1162, and checks that the product path refuses CPU
tensors instead of falling back to a CPU implementation.
"""
import inspect

import pytest
import torch

from chronicals_amd.kernels import cut_cross_entropy as cce


@pytest.mark.parametrize("V,d,gb,expect", [
    (50257, 768, 40.0, 4096),
    (100000, 4096, 40.0, 8192),
    (151936, 896, 40.0, 16384),
    (128256, 4096, 40.0, 16384),
    (151936, 896, 0.001, 256),          # VRAM cap, floor 256
    (151936, 8192, 0.5, 4096),          # 0.5*0.8 GiB / (8*8192 B) = 6553 -> 4096
])
def test_get_optimal_chunk_size(V, d, gb, expect):
    assert cce.get_optimal_chunk_size(V, d, gb) == expect


def test_estimate_memory_savings():
    r = cce.estimate_memory_savings(1, 8192, 151936, 8192)
    assert r["standard_mb"] == pytest.approx(8192 * 151936 * 8 / 2 ** 20)
    assert r["cce_mb"] == pytest.approx(8192 * 8192 * 8 / 2 ** 20)
    assert r["reduction_factor"] == pytest.approx(151936 / 8192)
    assert r["savings_mb"] == pytest.approx(r["standard_mb"] - r["cce_mb"])


def test_signature_matches_reference_order():
    params = list(inspect.signature(cce.cut_cross_entropy).parameters)
    assert params[:9] == ["hidden", "weight", "labels", "bias", "chunk_size", "ignore_index", "label_smoothing",
                          "z_loss_weight", "use_triton"]
    assert "reduction" in params
    sig = inspect.signature(cce.cut_cross_entropy)
    assert sig.parameters["chunk_size"].default == 8192
    assert sig.parameters["ignore_index"].default == -100
    assert sig.parameters["reduction"].default == "mean"


def test_loss_module_accepts_all_reductions_and_rejects_others():
    for red in ("mean", "sum", "none"):
        m = cce.CutCrossEntropyLoss(reduction=red)
        assert m.reduction == red
    with pytest.raises(ValueError):
        cce.CutCrossEntropyLoss(reduction="avg")
    m = cce.CutCrossEntropyLoss(chunk_size=4096, z_loss_weight=1e-4)
    assert m.extra_repr() == "chunk_size=4096, ignore_index=-100, label_smoothing=0.0, z_loss_weight=0.0001"


def test_reference_constants():
    assert (cce.CHUNK_SIZE_SMALL_VOCAB, cce.CHUNK_SIZE_MEDIUM_VOCAB, cce.CHUNK_SIZE_LARGE_VOCAB) == (4096, 8192, 16384)
    assert cce.DEFAULT_VOCAB_CHUNK_SIZE == 8192
    assert cce.TRITON_BLOCK_SIZE_MAX == 32768


def test_cpu_tensors_are_refused_not_computed():
    h = torch.randn(4, 8)
    w = torch.randn(10, 8)
    lab = torch.zeros(4, dtype=torch.long)
    with pytest.raises(RuntimeError, match="HIP devices"):
        cce.cut_cross_entropy(h, w, lab)
    with pytest.raises(RuntimeError, match="HIP devices"):
        cce.CutCrossEntropyLoss()(h, w, lab)


def test_bad_reduction_rejected_before_compute():
    with pytest.raises(ValueError):
        cce.cut_cross_entropy(torch.randn(2, 8), torch.randn(3, 8), torch.zeros(2, dtype=torch.long),
                              reduction="max")


def test_package_does_not_import_oracle():
    import pathlib
    root = pathlib.Path(cce.__file__).resolve().parents[1]
    for py in root.rglob("*.py"):
        text = py.read_text()
        for pat in ("import oracle", "from oracle", "cce_oracle"):
            assert pat not in text, f"{py} reaches the oracle ({pat})"


# ---------------------------------------------------------------------------
# torch.library registration (chronicals_amd/ops.py)
# ---------------------------------------------------------------------------

def test_custom_ops_registered():
    import chronicals_amd.ops  # noqa: F401
    assert hasattr(torch.ops.chronicals_hip, "cce_fwd")
    assert hasattr(torch.ops.chronicals_hip, "cce_bwd")


@pytest.mark.parametrize("reduction,loss_shape", [(0, (300,)), (1, (1,)), (2, (1,))])
def test_custom_op_fake_shapes_forward(reduction, loss_shape):
    import chronicals_amd.ops  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        h = torch.empty(300, 128, dtype=torch.bfloat16, device="cuda")
        w = torch.empty(1000, 128, dtype=torch.bfloat16, device="cuda")
        lab = torch.empty(300, dtype=torch.int64, device="cuda")
        loss, lse, nv, tgt = torch.ops.chronicals_hip.cce_fwd(h, w, lab, None, -100, 0.0, 0.0, 0, reduction)
        assert tuple(tgt.shape) == (300,) and tgt.dtype == torch.float32
        assert tuple(loss.shape) == loss_shape and loss.dtype == torch.float32
        assert tuple(lse.shape) == (300,) and lse.dtype == torch.float32
        assert tuple(nv.shape) == (1,) and nv.dtype == torch.int32


@pytest.mark.parametrize("need", [(True, True, True), (True, False, False), (False, True, False), (False, False, True)])
@pytest.mark.parametrize("f32", [False, True])
def test_custom_op_fake_shapes_backward(need, f32):
    import chronicals_amd.ops  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    need_dh, need_dw, need_db = need
    with FakeTensorMode():
        h = torch.empty(300, 128, dtype=torch.bfloat16, device="cuda")
        w = torch.empty(1000, 128, dtype=torch.bfloat16, device="cuda")
        lab = torch.empty(300, dtype=torch.int64, device="cuda")
        b = torch.empty(1000, dtype=torch.float32, device="cuda")
        lse = torch.empty(300, dtype=torch.float32, device="cuda")
        nv = torch.empty(1, dtype=torch.int32, device="cuda")
        g = torch.empty((), dtype=torch.float32, device="cuda")
        dh, dw, db = torch.ops.chronicals_hip.cce_bwd(g, h, w, lab, lse, nv, b, -100, 0.0, 0.0, 1, 8192,
                                                      need_dh, need_dw, need_db, f32, f32)
        gd = torch.float32 if f32 else torch.bfloat16
        assert tuple(dh.shape) == ((300, 128) if need_dh else (0,)) and dh.dtype == gd
        assert tuple(dw.shape) == ((1000, 128) if need_dw else (0,)) and dw.dtype == gd
        assert tuple(db.shape) == ((1000,) if need_db else (0,)) and db.dtype == torch.float32


def test_custom_op_has_no_cpu_kernel():
    import chronicals_amd.ops  # noqa: F401
    with pytest.raises(NotImplementedError):
        torch.ops.chronicals_hip.cce_fwd(torch.zeros(4, 8, dtype=torch.bfloat16), torch.zeros(5, 8, dtype=torch.bfloat16),
                                         torch.zeros(4, dtype=torch.int64), None, -100, 0.0, 0.0, 0, 1)


# ---------------------------------------------------------------------------
# Logits-in cross-entropy (chronicals_amd/kernels/logits_cross_entropy.py)
# ---------------------------------------------------------------------------

def test_logits_api_signatures_match_reference():
    from chronicals_amd.kernels import logits_cross_entropy as lce
    sig = lambda f: list(inspect.signature(f).parameters)  # noqa: E731
    # cut_cross_entropy.py:1169-1176 (+ reduction)
    assert sig(lce.chunked_cross_entropy_loss)[:6] == ["logits", "labels", "chunk_size", "ignore_index",
                                                       "label_smoothing", "z_loss_weight"]
    # triton_kernels.py:2979-2987, :3109-3116, :213-219
    assert sig(lce.liger_cross_entropy_forward) == ["logits", "target", "ignore_index", "lse_square_scale",
                                                    "label_smoothing", "reduction", "compute_grads"]
    assert sig(lce.liger_cross_entropy) == ["logits", "target", "ignore_index", "lse_square_scale",
                                            "label_smoothing", "reduction"]
    assert sig(lce.fused_cross_entropy) == ["logits", "labels", "label_smoothing", "z_loss_weight", "ignore_index"]
    assert inspect.signature(lce.fused_cross_entropy).parameters["z_loss_weight"].default == 1e-4
    # sequence_packer.py:1660-1667, sequence_packer_v2.py:1058-1065
    for f in (lce.compute_padding_free_loss, lce.compute_packed_loss):
        assert sig(f) == ["logits", "labels", "loss_mask", "ignore_index", "reduction", "label_smoothing"]
    m = lce.ChunkedCrossEntropyLoss()
    assert (m.chunk_size, m.ignore_index, m.label_smoothing, m.z_loss_weight) == (8192, -100, 0.0, 0.0)
    assert cce.chunked_cross_entropy_loss is lce.chunked_cross_entropy_loss
    assert cce.ChunkedCrossEntropyLoss is lce.ChunkedCrossEntropyLoss


def test_logits_apis_refuse_cpu_tensors():
    from chronicals_amd.kernels import logits_cross_entropy as lce
    x = torch.randn(2, 3, 10)
    lab = torch.zeros(2, 3, dtype=torch.long)
    for call in (lambda: lce.chunked_cross_entropy_loss(x, lab),
                 lambda: lce.liger_cross_entropy(x, lab),
                 lambda: lce.liger_cross_entropy_forward(x, lab),
                 lambda: lce.fused_cross_entropy(x, lab),
                 lambda: lce.compute_padding_free_loss(x, lab),
                 lambda: lce.compute_packed_loss(x, lab, torch.ones(2, 3))):
        with pytest.raises(RuntimeError, match="HIP devices"):
            call()


def test_logits_ops_fake_shapes():
    import chronicals_amd.ops  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(300, 1000, dtype=torch.float16, device="cuda")
        lab = torch.empty(300, dtype=torch.int64, device="cuda")
        for red, shape in ((0, (300,)), (1, (1,)), (2, (1,))):
            loss, lse, nv = torch.ops.chronicals_hip.ce_logits_fwd(x, lab, -100, 0.1, 0.0, 1, red)
            assert tuple(loss.shape) == shape and loss.dtype == torch.float32
            assert tuple(lse.shape) == (300,) and tuple(nv.shape) == (1,) and nv.dtype == torch.int32
        for f32, dt in ((False, torch.float16), (True, torch.float32)):
            g = torch.ops.chronicals_hip.ce_logits_bwd(loss, x, lab, lse, nv, -100, 0.1, 0.0, 1, 1, f32)
            assert tuple(g.shape) == (300, 1000) and g.dtype == dt


def test_logits_ops_have_no_cpu_kernel():
    import chronicals_amd.ops  # noqa: F401
    with pytest.raises(NotImplementedError):
        torch.ops.chronicals_hip.ce_logits_fwd(torch.zeros(4, 8), torch.zeros(4, dtype=torch.int64), -100, 0.0, 0.0,
                                               0, 1)


# ---------------------------------------------------------------------------
# Sibling fused linear-CE APIs (chronicals_amd/kernels/fused_linear_cross_entropy.py)
# ---------------------------------------------------------------------------

def test_fused_linear_api_signatures_match_reference():
    from chronicals_amd.kernels import fused_linear_cross_entropy as fl
    sig = lambda f: list(inspect.signature(f).parameters)  # noqa: E731
    # triton_kernels.py:2308-2315, :2398-2408, :2636-2645, :2659-2666
    assert sig(fl.fused_linear_cross_entropy_forward) == ["hidden", "weight", "labels", "bias", "chunk_size",
                                                          "ignore_index"]
    assert sig(fl.fused_linear_cross_entropy) == ["hidden", "weight", "labels", "bias", "label_smoothing",
                                                  "z_loss_weight", "ignore_index", "chunk_size", "reduction"]
    assert sig(fl.fused_linear_cross_entropy_autograd) == ["hidden", "weight", "labels", "bias", "label_smoothing",
                                                           "z_loss_weight", "ignore_index", "chunk_size"]
    assert sig(fl.chunked_cross_entropy) == ["logits", "labels", "chunk_size", "label_smoothing", "z_loss_weight",
                                             "ignore_index"]
    assert inspect.signature(fl.fused_linear_cross_entropy).parameters["z_loss_weight"].default == 1e-4
    assert inspect.signature(fl.chunked_cross_entropy).parameters["z_loss_weight"].default == 1e-4
    # :3147-3157, :3318-3328
    for f in (fl.triton_fused_linear_cross_entropy_forward, fl.triton_fused_linear_cross_entropy):
        assert sig(f) == ["hidden", "weight", "target", "bias", "ignore_index", "lse_square_scale",
                          "label_smoothing", "reduction", "chunk_size"]
    assert sig(fl.FusedLinearCrossEntropyLoss.forward) == ["self", "hidden", "weight", "bias", "labels"]
    assert sig(fl.TritonFusedLinearCrossEntropyLoss.forward) == ["self", "hidden", "weight", "target", "bias"]
    m = fl.FusedLinearCrossEntropyLoss()
    assert (m.chunk_size, m.label_smoothing, m.z_loss_weight, m.ignore_index) == (8192, 0.0, 1e-4, -100)
    t = fl.TritonFusedLinearCrossEntropyLoss()
    assert (t.chunk_size, t.ignore_index, t.lse_square_scale, t.label_smoothing, t.reduction) == (
        8192, -100, 0.0, 0.0, "mean")
    assert fl.ChunkedCrossEntropyLoss is fl.FusedLinearCrossEntropyLoss
    assert fl.LigerFusedLinearCrossEntropyLoss is fl.TritonFusedLinearCrossEntropyLoss
    assert fl.DEFAULT_CHUNK_SIZE == 8192


def test_fused_linear_apis_refuse_cpu_tensors():
    from chronicals_amd.kernels import fused_linear_cross_entropy as fl
    h, w, lab = torch.randn(4, 8), torch.randn(10, 8), torch.zeros(4, dtype=torch.long)
    for call in (lambda: fl.fused_linear_cross_entropy(h, w, lab),
                 lambda: fl.fused_linear_cross_entropy_autograd(h, w, lab),
                 lambda: fl.FusedLinearCrossEntropyLoss()(h, w, None, lab),
                 lambda: fl.triton_fused_linear_cross_entropy(h, w, lab),
                 lambda: fl.triton_fused_linear_cross_entropy_forward(h, w, lab),
                 lambda: fl.fused_linear_cross_entropy_forward(h, w, lab),
                 lambda: fl.chunked_cross_entropy(torch.randn(1, 4, 10), lab.view(1, 4))):
        with pytest.raises(RuntimeError, match="HIP devices"):
            call()


def test_reference_module_public_names_all_present():
    # every public name of chronicals/kernels/cut_cross_entropy.py (:47-1430)
    for name in ("CHUNK_SIZE_SMALL_VOCAB", "CHUNK_SIZE_MEDIUM_VOCAB", "CHUNK_SIZE_LARGE_VOCAB",
                 "DEFAULT_VOCAB_CHUNK_SIZE", "TRITON_BLOCK_SIZE", "TRITON_BLOCK_SIZE_MAX", "get_optimal_chunk_size",
                 "CutCrossEntropyForward", "CutCrossEntropyBackward", "CutCrossEntropyFunction", "cut_cross_entropy",
                 "CutCrossEntropyLoss", "chunked_cross_entropy_loss", "ChunkedCrossEntropyLoss",
                 "AdaptiveCrossEntropyLoss", "compute_z_loss", "estimate_memory_savings"):
        assert hasattr(cce, name), name
    sig = lambda f: list(inspect.signature(f).parameters)  # noqa: E731
    assert sig(cce.CutCrossEntropyForward.forward) == ["hidden", "weight", "labels", "bias", "chunk_size",
                                                       "ignore_index", "label_smoothing", "z_loss_weight",
                                                       "use_kahan"]
    assert sig(cce.CutCrossEntropyBackward.backward) == ["hidden", "weight", "labels", "logsumexp", "valid_mask",
                                                         "grad_output", "bias", "chunk_size", "ignore_index",
                                                         "label_smoothing", "z_loss_weight"]
    a = cce.AdaptiveCrossEntropyLoss()
    assert (a.small_vocab_threshold, a.large_vocab_threshold, a.ignore_index, a.label_smoothing,
            a.z_loss_weight) == (32000, 100000, -100, 0.0, 0.0)
    with pytest.raises(RuntimeError, match="HIP devices"):
        a(torch.randn(4, 8), torch.randn(40000, 8), torch.zeros(4, dtype=torch.long))


def test_reference_import_blocks_resolve():
    # the names chronicals_trainer.py:79-89 and triton_kernels.py:44-58 import
    # from the reference module; with this package's module path they resolve
    from chronicals_amd.kernels.cut_cross_entropy import (  # noqa: F401
        CutCrossEntropyFunction,
        CutCrossEntropyLoss,
        DEFAULT_VOCAB_CHUNK_SIZE,
        cce_backward_pytorch,
        cce_forward_pytorch,
        cut_cross_entropy,
        estimate_memory_savings,
        get_optimal_chunk_size,
        linear_cross_entropy,
    )
    assert cce_forward_pytorch is cce.CutCrossEntropyForward.forward
    assert cce_backward_pytorch is cce.CutCrossEntropyBackward.backward
    sig = list(inspect.signature(linear_cross_entropy).parameters)
    assert sig[:6] == ["hidden", "weight", "labels", "bias", "ignore_index", "reduction"]
    with pytest.raises(RuntimeError, match="HIP devices"):
        linear_cross_entropy(torch.randn(4, 8), torch.randn(10, 8), torch.zeros(4, dtype=torch.long))
    with pytest.raises(ValueError):
        linear_cross_entropy(torch.randn(4, 8), torch.randn(10, 8), torch.zeros(4, dtype=torch.long),
                             reduction="avg")
