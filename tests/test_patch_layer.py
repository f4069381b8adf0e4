"""CPU tests of the patch layer (``pymsst_amd.fused_roformer``), mirroring the reference's
switchboard tests (tests/test_training_smoke.py:236-512, 627-637): backend and mode
normalisation, fallback when the extension is missing, duck-typed ``extension=``
injection, bwd-mode precedence, the layout-reduce-copy helpers, the packing autograd
Function, the pure-torch GLU Function, parameter-reference caches, and that every
patch can be undone."""

from __future__ import annotations

import pytest
import torch

from pymsst_amd import fused_roformer as fr
from pymsst_amd.core import bands, common, transformer
from pymsst_amd.core.bs_roformer import BSRoformer

_BANDS = (2,) * 16 + (4,) * 8 + (32,) + (33,)


def _small_model(mask_depth: int = 2) -> BSRoformer:
    torch.manual_seed(0)
    return BSRoformer(dim=16, depth=1, stereo=True, num_stems=1, heads=2, dim_head=8, stft_n_fft=256,
                      stft_hop_length=64, stft_win_length=256, freqs_per_bands=_BANDS,
                      mask_estimator_depth=mask_depth, mlp_expansion_factor=2, loss="spec_l1")


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    for name in list(fr.RUNTIME_PRESETS["hip_full"]) + [fr.EXPERIMENTAL_RMS_NORM_ENV, fr.EXPERIMENTAL_GROUPED_LINEAR_ENV,
                                                         fr.EXPERIMENTAL_MASK_ESTIMATOR_FINAL_ENV,
                                                         fr.EXPERIMENTAL_BAND_SPLIT_BWD_V2_ENV,
                                                         fr.EXPERIMENTAL_TRAIN_PARAM_PACK_AUTOGRAD_ENV,
                                                         fr.EXPERIMENTAL_ATTENTION_GATES_ENV]:
        monkeypatch.delenv(name, raising=False)
    monkeypatch.setenv(fr.CORE_GROUPED_TRAIN_ENV, "")
    yield
    fr.restore_stock_implementations()


def test_backend_defaults_to_off():
    status = fr.apply_roformer_fused_training_backend(_small_model(), None)
    assert status.active == "off" and status.requested == "off" and status.reason is None
    assert fr.normalize_fused_kernel_backend("CUDA-EXT") == "cuda_ext"
    assert fr.normalize_fused_kernel_backend("hip") == "cuda_ext"
    with pytest.raises(ValueError, match="fused_kernel_backend"):
        fr.normalize_fused_kernel_backend("unknown")
    with pytest.raises(ValueError, match="fused_rms_norm_mode"):
        fr.normalize_fused_rms_norm_mode("unknown")


def test_falls_back_when_extension_is_unavailable(monkeypatch):
    def fail_load():
        raise fr.FusedKernelUnavailable("no extension in this test")

    monkeypatch.setattr(fr, "load_fused_band_split_extension", fail_load)
    with pytest.warns(RuntimeWarning, match="no extension"):
        status = fr.apply_roformer_fused_training_backend(_small_model(), "cuda_ext")
    assert status.active == "off" and status.requested == "cuda_ext"
    assert "no extension" in status.reason


def test_real_loader_refuses_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(fr.FusedKernelUnavailable):
        fr.load_fused_band_split_extension()


def test_can_patch_band_split_with_injected_extension():
    model = _small_model()
    status = fr.apply_roformer_fused_training_backend(model, "cuda_ext", extension=object())
    assert status.active == "cuda_ext" and status.patched_band_splits == 1
    assert model.band_split._pymsst_fused_band_split is True
    assert status.patched_single_stem_masks is True
    # patching twice is idempotent
    again = fr.apply_roformer_fused_training_backend(model, "cuda_ext", extension=object())
    assert again.patched_band_splits == 0


def test_band_split_bwd_v3_takes_precedence_over_v2(monkeypatch):
    class FakeExtension:
        def band_split_backward_v2(self):
            raise AssertionError("not called")

        def band_split_backward_v3(self):
            raise AssertionError("not called")

    monkeypatch.setenv(fr.EXPERIMENTAL_BAND_SPLIT_BWD_V2_ENV, "1")
    monkeypatch.setenv(fr.EXPERIMENTAL_BAND_SPLIT_BWD_V3_ENV, "1")
    model = _small_model()
    status = fr.apply_roformer_fused_training_backend(model, "cuda_ext", extension=FakeExtension())
    assert status.patched_band_split_bwd_v2 is False and status.patched_band_split_bwd_v3 is True
    assert model.band_split._pymsst_fused_band_split_bwd_mode == "v3"


def test_rms_norm_bwd_v2_env_enables_fast_mode(monkeypatch):
    assert fr.normalize_fused_rms_norm_mode(None) is None
    monkeypatch.setenv(fr.EXPERIMENTAL_RMS_NORM_BWD_V2_ENV, "1")
    assert fr.normalize_fused_rms_norm_mode(None) == "fast"
    assert fr.normalize_fused_rms_norm_mode("off") is None
    monkeypatch.setenv(fr.EXPERIMENTAL_RMS_NORM_ENV, "safe")
    assert fr.normalize_fused_rms_norm_mode(None) == "mixed"


def test_status_records_every_patch_with_full_extension(monkeypatch):
    ext = type("FullExt", (), {name: object() for name in (
        "band_split_forward", "band_split_backward", "band_split_backward_v2", "band_split_backward_v3",
        "band_split_ragged_forward", "band_split_ragged_backward", "grouped_linear_forward", "rotary_forward",
        "rotary_backward", "rms_norm_forward", "rms_norm_backward", "rms_norm_forward_fp32_gamma",
        "rms_norm_backward_fp32_gamma", "rms_norm_forward_mixed", "rms_norm_backward_mixed",
        "mask_estimator_final_forward", "mask_estimator_final_backward", "mask_estimator_final_direct_forward",
        "mask_estimator_final_direct_backward")})()
    for key, value in fr.RUNTIME_PRESETS["hip_full"].items():
        monkeypatch.setenv(key, value)
    monkeypatch.setenv(fr.EXPERIMENTAL_TRAIN_PARAM_PACK_AUTOGRAD_ENV, "1")
    status = fr.apply_roformer_fused_training_backend(_small_model(), "hip", extension=ext)
    assert status.patched_band_split_ragged_forward and status.patched_band_split_ragged_backward
    assert status.patched_band_split_bwd_v3 and status.patched_rotary
    assert status.patched_rms_norm and status.rms_norm_mode == "fast" and status.patched_rms_norm_bwd_v2
    assert status.patched_layout_reduce_copy and status.patched_mask_final_autograd
    assert status.patched_train_param_pack_autograd
    assert status.patched_mask_estimator_final and status.mask_estimator_final_mode == "direct"
    assert status.patched_attention_gates is False
    assert getattr(transformer.apply_rotary_emb_fast, "_pymsst_fused_rotary", False)
    assert getattr(transformer.RMSNorm.forward, "_pymsst_fused_rms_norm", False)


def test_restore_stock_implementations_unwinds_everything(monkeypatch):
    originals = (transformer.apply_rotary_emb_fast, transformer.RMSNorm.forward, bands.grouped_linear,
                 bands.MaskEstimator._forward_layer_grouped_mlp, bands.MaskEstimator._get_layer_group_params,
                 bands.BandSplit._get_group_params, common.RoformerRuntimeMixin._estimate_masks)
    ext = type("Ext", (), {n: object() for n in ("rotary_forward", "rotary_backward", "rms_norm_forward",
                                                  "rms_norm_backward", "grouped_linear_forward",
                                                  "mask_estimator_final_direct_forward",
                                                  "mask_estimator_final_direct_backward")})()
    for key, value in fr.RUNTIME_PRESETS["hip_full"].items():
        monkeypatch.setenv(key, value)
    monkeypatch.setenv(fr.EXPERIMENTAL_GROUPED_LINEAR_ENV, "1")
    model = _small_model()
    fr.apply_roformer_fused_training_backend(model, "hip", extension=ext, rms_norm_mode="fast")
    assert transformer.apply_rotary_emb_fast is not originals[0]
    assert bands.grouped_linear is not originals[2]
    fr.restore_stock_implementations(model)
    now = (transformer.apply_rotary_emb_fast, transformer.RMSNorm.forward, bands.grouped_linear,
           bands.MaskEstimator._forward_layer_grouped_mlp, bands.MaskEstimator._get_layer_group_params,
           bands.BandSplit._get_group_params, common.RoformerRuntimeMixin._estimate_masks)
    assert all(a is b for a, b in zip(originals, now))
    assert "_forward_grouped" not in model.band_split.__dict__
    assert not getattr(model.band_split, "_pymsst_fused_band_split", False)


def test_band_selection_narrows_runs_and_gathers_the_rest():
    x = torch.arange(2 * 4 * 3, dtype=torch.float32).reshape(2, 4, 3)
    est = _small_model().mask_estimators[0]
    assert fr._run_of((1, 2)) == (1, 3) and fr._run_of((0, 2)) is None and fr._run_of(()) is None
    run = fr._bands_of(est, x, (1, 2))
    assert run._base is not None and torch.equal(run, x[..., 1:3, :])  # a view, no gather
    assert torch.equal(fr._bands_of(est, x, (0, 2)), x.index_select(-2, torch.tensor((0, 2))))


@pytest.mark.parametrize("mask_depth", [2, 3])
def test_layout_reduce_copy_matches_original_mask_mlp(monkeypatch, mask_depth):
    monkeypatch.setenv(fr.EXPERIMENTAL_LAYOUT_REDUCE_COPY_ENV, "1")
    model = _small_model(mask_depth)
    estimator = model.mask_estimators[0]
    x = torch.randn(2, len(estimator.dim_inputs), 16)
    reference = bands.MaskEstimator._forward_layer_grouped_mlp(estimator, x)
    status = fr.apply_roformer_fused_training_backend(model, "cuda_ext", extension=object())
    candidate = estimator._forward_layer_grouped_mlp(x)
    assert status.patched_layout_reduce_copy is True
    assert reference is not None and candidate is not None
    assert torch.equal(candidate, reference)


def test_flat_params_views_match_stack_and_cast():
    """A packed run of parameters, cast to fp16, equals ``stack([p.to(fp16)])`` and its backward gives each
    parameter its slice of the gradient in the parameter's dtype; the parameters keep their identity and
    become views of one storage."""
    from pymsst_amd.packed_params import FlatParams

    params = [torch.nn.Parameter(torch.randn(2, 3)) for _ in range(4)]
    refs = [p.detach().clone().requires_grad_() for p in params]
    ids = [id(p) for p in params]
    pk = FlatParams(params)
    assert [id(p) for p in params] == ids and pk.intact()
    assert all(p.data_ptr() == pk.storage.data_ptr() + 6 * 4 * i for i, p in enumerate(params))
    grad = torch.randn(3, 2, 3, dtype=torch.float16)
    got = pk.group(1, 4, torch.float16)
    want = torch.stack([r.to(torch.float16) for r in refs[1:]], dim=0)
    assert torch.equal(got, want)
    got.backward(grad)
    want.backward(grad)
    assert params[0].grad is None
    for p, r in zip(params[1:], refs[1:]):
        assert p.grad.dtype == torch.float32 and torch.equal(p.grad, r.grad)
    flat = pk.flat()
    assert torch.equal(flat, torch.cat([r.detach().reshape(-1) for r in refs]))


def test_flat_params_cast_follows_optimizer_updates_and_device_moves():
    from pymsst_amd.packed_params import FlatParams, pack

    mod = torch.nn.Module()
    params = [torch.nn.Parameter(torch.randn(5)) for _ in range(3)]
    pk = pack(mod, "k", params)
    assert pack(mod, "k", params) is pk
    c1 = pk.flat(torch.bfloat16).detach().clone()
    opt = torch.optim.SGD(params, lr=1.0)
    for p in params:
        p.grad = torch.ones_like(p)
    opt.step()
    c2 = pk.flat(torch.bfloat16)
    assert not torch.equal(c2, c1)  # the cached cast was refreshed
    assert torch.equal(c2, torch.cat([p.detach() for p in params]).bfloat16())
    params[1].data = params[1].data.clone()  # no longer a view of the storage (what .to() does)
    assert not pk.intact()
    pk2 = pack(mod, "k", params)
    assert pk2 is not pk and pk2.intact() and isinstance(pk2, FlatParams)


def _spec_batch(model):
    g = torch.Generator().manual_seed(1)
    mix = 0.1 * torch.randn(1, 2, 2048, generator=g)
    return mix, 0.1 * torch.randn(1, 1, 2, 2048, generator=g)


@pytest.mark.parametrize("first", ["inference", "train"])
def test_packed_params_survive_inference_mode_validation(monkeypatch, first):
    """The packs and their casts are normal tensors even when first built under torch.inference_mode()
    (a validation pass): a train step after an inference-mode pass, and one before it, both work, and a
    cast made during the inference pass is not handed to the training step."""
    monkeypatch.setenv(fr.EXPERIMENTAL_LAYOUT_REDUCE_COPY_ENV, "1")
    model = _small_model()
    fr.apply_roformer_fused_training_backend(model, "cuda_ext", extension=object())
    mix, target = _spec_batch(model)

    def validate():
        model.eval()
        with torch.no_grad():  # an optimizer-like update: the next cast request misses the cache
            model.band_split.to_features[0][1].weight.add_(0.0)
        with torch.inference_mode():
            model(mix)
            # a bf16 cast made in inference mode
            bs = model.band_split
            bs._get_group_params(0, 2, torch.device("cpu"), torch.bfloat16)
        model.train()

    def train_step():
        model.train()
        model(mix, target).backward()
        bs = model.band_split
        w = bs._get_group_params(0, 2, torch.device("cpu"), torch.bfloat16)[1]
        assert not w.is_inference()
        w.float().sum().backward()  # the cached cast is saved for backward without error

    steps = [validate, train_step, validate, train_step] if first == "inference" else [train_step, validate, train_step]
    for fn in steps:
        fn()
    packs = model.band_split.__dict__["_pymsst_packs"]
    assert packs and not any(fp.storage.is_inference() for fp in packs.values())
    assert all(not p.is_inference() for p in model.parameters())


def test_flat_params_cast_follows_storage_writes_and_invalidate():
    """A write to the shared storage refreshes the cached cast by itself; a write through ``param.data``
    bypasses every version counter and needs ``invalidate``."""
    from pymsst_amd.packed_params import FlatParams, invalidate_casts

    params = [torch.nn.Parameter(torch.randn(4)) for _ in range(2)]
    pk = FlatParams(params)
    c1 = pk.flat(torch.bfloat16).detach().clone()
    with torch.no_grad():
        pk.storage.mul_(2)
    c2 = pk.flat(torch.bfloat16).detach().clone()
    assert torch.equal(c2, (2 * c1.float()).bfloat16())
    params[0].data.add_(1)
    assert torch.equal(pk.flat(torch.bfloat16), c2)  # stale: documented
    mod = torch.nn.Module()
    mod.__dict__["_pymsst_packs"] = {"k": pk}
    invalidate_casts(mod)
    assert torch.equal(pk.flat(torch.bfloat16), torch.cat([p.detach() for p in params]).bfloat16())


def test_packed_band_split_keeps_state_dict_and_is_zero_copy(monkeypatch):
    monkeypatch.setenv(fr.EXPERIMENTAL_LAYOUT_REDUCE_COPY_ENV, "1")
    model = _small_model()
    keys = list(model.state_dict())
    ref = {k: v.clone() for k, v in model.state_dict().items()}
    bs = model.band_split
    stock = bands.BandSplit._get_group_params(bs, 0, 2, torch.device("cpu"), torch.float32)
    fr.apply_roformer_fused_training_backend(model, "cuda_ext", extension=object())
    got = bs._get_group_params(0, 2, torch.device("cpu"), torch.float32)
    assert all(torch.equal(a, b) for a, b in zip(got, stock))
    gamma_pack = bs.__dict__["_pymsst_packs"]["band_split.gamma"]
    assert got[0].data_ptr() == gamma_pack.storage.data_ptr()  # a view of the storage, not a stack
    assert list(model.state_dict()) == keys
    assert all(torch.equal(v, ref[k]) for k, v in model.state_dict().items())
    fr.restore_stock_implementations(model)


def _reference_grouped_linear(x, weight, bias):
    """bmm / baddbmm per group (tests/test_training_smoke.py:28-37 semantics)."""
    g, _, i = weight.shape
    lead = x.shape[:-2]
    x3 = x.reshape(-1, g, i).transpose(0, 1)
    wt = weight.transpose(1, 2).contiguous()
    out = torch.bmm(x3, wt) if bias is None else torch.baddbmm(bias.unsqueeze(1).expand(-1, x3.shape[1], -1), x3, wt)
    return out.transpose(0, 1).reshape(*lead, g, -1)


def test_mask_final_grouped_linear_glu_matches_reference():
    torch.manual_seed(3)
    x = torch.randn(2, 5, 3, 4, requires_grad=True)
    weight = torch.randn(3, 6, 4, requires_grad=True)
    bias = torch.randn(3, 6, requires_grad=True)
    rx, rw, rb = (t.detach().clone().requires_grad_() for t in (x, weight, bias))
    grad = torch.randn(2, 5, 3, 3)
    out = fr._MaskFinalGroupedLinearGLU.apply(x, weight, bias)
    ref = torch.nn.functional.glu(_reference_grouped_linear(rx, rw, rb), dim=-1)
    out.backward(grad)
    ref.backward(grad)
    assert torch.allclose(out, ref)
    for a, b in ((x, rx), (weight, rw), (bias, rb)):
        assert torch.allclose(a.grad, b.grad, atol=1e-6, rtol=1e-6)


def test_grouped_mlp_forward_restores_band_order_for_interleaved_groups(monkeypatch):
    """Widths whose equal-signature bands are not runs (8, 16, 8, 16): the final layer's groups are
    gathered with index_select and the outputs come back in band order, equal to the per-band MLPs."""
    monkeypatch.setenv(fr.EXPERIMENTAL_LAYOUT_REDUCE_COPY_ENV, "1")
    torch.manual_seed(5)
    est = bands.MaskEstimator(16, (8, 16, 8, 16), depth=2, mlp_expansion_factor=2)
    x = torch.randn(3, 4, 16)
    per_band = torch.cat([mlp(xb) for xb, mlp in zip(x.unbind(dim=-2), est.to_freqs)], dim=-1)
    fr._patch_core_packed_params()
    try:
        got = est._forward_layer_grouped_mlp(x)
    finally:
        fr.restore_stock_implementations()
    assert torch.allclose(got, per_band, atol=1e-6, rtol=1e-6)


def test_cpu_inputs_take_the_stock_path_after_patching(monkeypatch):
    """Patched functions keep the stock behaviour for inputs the kernels do not take (CPU
    tensors): a patched CPU model computes exactly what the unpatched one does."""
    for key, value in fr.RUNTIME_PRESETS["hip_full"].items():
        monkeypatch.setenv(key, value)
    ext = type("Ext", (), {n: object() for n in ("rotary_forward", "rotary_backward", "rms_norm_forward",
                                                  "rms_norm_backward", "band_split_ragged_forward",
                                                  "band_split_ragged_backward",
                                                  "mask_estimator_final_direct_forward",
                                                  "mask_estimator_final_direct_backward")})()
    model = _small_model()
    model.train()
    mixture = torch.randn(1, 2, 2048) * 0.1
    target = torch.randn(1, 1, 2, 2048) * 0.1
    monkeypatch.setenv(fr.CORE_GROUPED_TRAIN_ENV, "1")
    ref = model(mixture, target)
    fr.apply_roformer_fused_training_backend(model, "hip", extension=ext, rms_norm_mode="fast")
    got = model(mixture, target)
    assert torch.equal(got, ref)


class _OracleGateExt:
    """CPU stand-in with the attention-gate op names, computing through the numpy oracle."""

    def __init__(self, bnhd: bool):
        if bnhd:
            self.attention_gate_forward_bnhd = self._fwd4
            self.attention_gate_backward_bnhd = self._bwd4

    @staticmethod
    def _np(t):
        return t.detach().double().numpy()

    def attention_gate_forward(self, attn, x, weight, bias):
        import oracle

        out, gate = oracle.attention_gate_forward(self._np(attn), self._np(x), self._np(weight), self._np(bias), "f64")
        return [torch.from_numpy(out), torch.from_numpy(gate), attn, x]

    def attention_gate_backward(self, grad_out, attn, x, weight, gate):
        import oracle

        res = oracle.attention_gate_backward(self._np(grad_out), self._np(attn), self._np(x), self._np(weight),
                                             self._np(gate), "f64")
        return [torch.from_numpy(r) for r in res]

    def _fwd4(self, attn, x, weight, bias):
        out, gate, _, _ = self.attention_gate_forward(attn.reshape(-1, *attn.shape[2:]), x, weight, bias)
        return [out, gate, attn, x]

    def _bwd4(self, grad_out, attn, x, weight, gate, out_layout="bhnd"):
        ga, gx, gw, gb = self.attention_gate_backward(grad_out, attn.reshape(-1, *attn.shape[2:]), x, weight, gate)
        return [ga.reshape(attn.shape), gx, gw, gb]


@pytest.mark.parametrize("bnhd", [False, True])
def test_fused_attention_gate_function_matches_autograd(bnhd):
    from tests import torch_reference as tr

    g = torch.Generator().manual_seed(3)
    b, n, h, dh, d = 2, 5, 4, 8, 12
    attn = torch.randn(b, h, n, dh, generator=g, dtype=torch.float64).transpose(1, 2).requires_grad_()
    x = torch.randn(b, n, d, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(h, d, generator=g, dtype=torch.float64, requires_grad=True)
    bias = torch.randn(h, generator=g, dtype=torch.float64, requires_grad=True)
    out = fr._FusedAttentionGate.apply(attn, x, w, bias, _OracleGateExt(bnhd))
    assert out.shape == (b, n, h * dh)
    gout = torch.randn(out.shape, generator=g, dtype=torch.float64)
    grads = torch.autograd.grad(out, (attn, x, w, bias), gout)
    ref = tr.attention_gate(attn.reshape(b * n, h, dh), x.reshape(b * n, d), w, bias).reshape(b, n, -1)
    torch.testing.assert_close(out, ref)
    rgrads = torch.autograd.grad(ref, (attn, x, w, bias), gout)
    for got, want in zip(grads, rgrads):
        torch.testing.assert_close(got, want)


def test_attention_gate_patch_and_restore(monkeypatch):
    original = transformer.Attention.forward
    ext = _OracleGateExt(True)
    monkeypatch.setenv(fr.EXPERIMENTAL_ATTENTION_GATES_ENV, "gate")
    status = fr.apply_roformer_fused_training_backend(_small_model(), "hip", extension=ext)
    assert status.patched_attention_gates and status.attention_gate_mode == "full"
    assert getattr(transformer.Attention.forward, "_pymsst_fused_attention_gates", False)
    fr.restore_stock_implementations()
    assert transformer.Attention.forward is original
    monkeypatch.setenv(fr.EXPERIMENTAL_ATTENTION_GATES_ENV, "off")
    status = fr.apply_roformer_fused_training_backend(_small_model(), "hip", extension=ext)
    assert not status.patched_attention_gates and status.attention_gate_mode is None


@pytest.mark.parametrize("bias", [True, False])
def test_stock_grouped_linear_explicit_backward_matches_autograd(bias):
    """The stock grouped_linear's hand-written backward (contiguous operands for every batched
    product) equals autograd of the same per-group Linear."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 5, 4, 6, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(4, 7, 6, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(4, 7, generator=g, dtype=torch.float64, requires_grad=True) if bias else None
    out = bands.grouped_linear(x, w, b)
    ref = torch.stack([x[..., k, :] @ w[k].T + (b[k] if bias else 0) for k in range(4)], dim=-2)
    torch.testing.assert_close(out, ref)
    gout = torch.randn(out.shape, generator=g, dtype=torch.float64)
    inputs = [t for t in (x, w, b) if t is not None]
    for got, want in zip(torch.autograd.grad(out, inputs, gout), torch.autograd.grad(ref, inputs, gout)):
        torch.testing.assert_close(got, want)
