"""Host-side API contracts (CPU): loader without fallback, operand normalisation,
GEMV/GEMM routing, and the static linear scheme's dispatch - the shape of the
reference's test_native_loader.py and test_static_scheme.py."""

import os
import types
from unittest.mock import patch

import pytest
import torch

from hif8_rocm import native
from hif8_rocm.scheme import STATIC_QUANT_TYPE, W8A8HiFloat8StaticLinearMethod


@pytest.fixture(autouse=True)
def _fresh_loader():
    native.reset_extension_cache()
    yield
    native.reset_extension_cache()


def test_missing_extension_raises_without_fallback():
    with patch("importlib.import_module", side_effect=ModuleNotFoundError("missing")):
        with pytest.raises(native.NativeExtensionUnavailable, match="no decoded-weight or floating-point fallback"):
            native.load_extension()
    # The failure is cached.
    with pytest.raises(native.NativeExtensionUnavailable):
        native.load_extension()


def test_missing_symbol_is_rejected():
    incomplete = types.SimpleNamespace(hif8_dynamic_quant=lambda *a: a, hif8_static_quant=lambda *a: a)
    with patch("importlib.import_module", return_value=incomplete):
        with pytest.raises(native.NativeExtensionUnavailable, match="soft_hif8_gemv"):
            native.load_extension()


def test_valid_extension_is_cached():
    complete = types.SimpleNamespace(hif8_dynamic_quant=lambda *a: a, hif8_static_quant=lambda *a: a,
                                     soft_hif8_gemv=lambda *a: a, soft_hif8_gemm=lambda *a: a)
    with patch("importlib.import_module", return_value=complete) as importer:
        assert native.load_extension() is complete
        assert native.load_extension() is complete
        importer.assert_called_once()


def test_real_extension_loads_on_cpu():
    ext = native.load_extension()
    for name in ("hif8_dynamic_quant", "hif8_static_quant", "hif8_scaled_decode", "soft_hif8_gemv",
                 "soft_hif8_gemm", "soft_hif8_static_fused_gemm", "soft_hif8_fused_gemm"):
        assert callable(getattr(ext, name))
        assert callable(getattr(torch.ops.vllm_ascend_hif8, name))
    for name in ("hif8_kv_cache_write", "hif8_paged_decode_attention", "hif8_embedding_lookup"):
        assert callable(getattr(torch.ops.vllm_ascend_hif8, name))


def test_meta_shapes():
    native.load_extension()
    x = torch.empty(3, 2, 64, dtype=torch.bfloat16, device="meta")
    data, scale = torch.ops.vllm_ascend_hif8.hif8_static_quant(x, torch.empty(1, device="meta"))
    assert data.shape == x.shape and data.dtype == torch.uint8
    assert scale.shape == (6,) and scale.dtype == torch.float32
    y = torch.ops.vllm_ascend_hif8.soft_hif8_gemm(
        torch.empty(5, 64, dtype=torch.uint8, device="meta"), torch.empty(7, 64, dtype=torch.uint8, device="meta"),
        torch.empty(5, device="meta"), torch.empty(7, device="meta"), None, torch.bfloat16)
    assert y.shape == (5, 7) and y.dtype == torch.bfloat16
    yd = torch.ops.vllm_ascend_hif8.soft_hif8_gemm_decoded_weight(
        torch.empty(5, 64, dtype=torch.uint8, device="meta"), torch.empty(7, 64, dtype=torch.bfloat16, device="meta"),
        torch.empty(5, device="meta"), torch.empty(7, device="meta"), None, torch.float16)
    assert yd.shape == (5, 7) and yd.dtype == torch.float16
    wd = torch.ops.vllm_ascend_hif8.hif8_decode_bf16(torch.empty(7, 64, dtype=torch.uint8, device="meta"))
    assert wd.shape == (7, 64) and wd.dtype == torch.bfloat16
    d, ds = torch.ops.vllm_ascend_hif8.hif8_dynamic_quant(x)
    assert d.shape == x.shape and d.dtype == torch.uint8 and ds.shape == (6,) and ds.dtype == torch.float32
    f = torch.ops.vllm_ascend_hif8.soft_hif8_fused_gemm(
        torch.empty(2, 64, dtype=torch.float16, device="meta"), torch.empty(7, 64, dtype=torch.uint8, device="meta"),
        torch.empty(7, device="meta"), None, torch.float16)
    assert f.shape == (2, 7) and f.dtype == torch.float16
    e = torch.ops.vllm_ascend_hif8.hif8_embedding_lookup(
        torch.empty(2, 3, dtype=torch.int64, device="meta"), torch.empty(50, 64, dtype=torch.uint8, device="meta"),
        torch.empty(50, device="meta"))
    assert e.shape == (2, 3, 64) and e.dtype == torch.bfloat16


def test_decode_glue_meta_shapes():
    native.load_extension()
    ops = torch.ops.vllm_ascend_hif8
    meta = dict(device="meta")
    h = torch.empty(3, 64, dtype=torch.bfloat16, **meta)
    w = torch.empty(64, dtype=torch.bfloat16, **meta)
    s = torch.empty(1, **meta)
    assert ops.hif8_add_rms_norm(h, None, w, 1e-6).shape == (3, 64)
    y, codes, rs = ops.hif8_add_rms_norm_quant(h, h, w, 1e-6, s)
    assert y.shape == (3, 64) and codes.dtype == torch.uint8 and codes.shape == (3, 64) and rs.shape == (3,)
    gu = torch.empty(2, 5, 96, dtype=torch.bfloat16, **meta)
    assert ops.hif8_silu_mul(gu).shape == (2, 5, 48)
    c2, r2 = ops.hif8_silu_mul_quant(gu, s)
    assert c2.shape == (2, 5, 48) and c2.dtype == torch.uint8 and r2.shape == (2, 5) and r2.dtype == torch.float32
    g = ops.hif8_bf16_gemv(torch.empty(4, 64, dtype=torch.bfloat16, **meta),
                           torch.empty(9, 64, dtype=torch.bfloat16, **meta))
    assert g.shape == (4, 9) and g.dtype == torch.bfloat16
    q, k, v, slots = ops.hif8_qk_norm_rope(
        torch.empty(2, (8 + 2 * 2) * 32, dtype=torch.bfloat16, **meta), torch.empty(32, dtype=torch.bfloat16, **meta),
        torch.empty(32, dtype=torch.bfloat16, **meta), torch.empty(2, dtype=torch.int64, **meta),
        torch.empty(8, **meta), torch.empty(2, 4, dtype=torch.int32, **meta), 16, 8, 2, 32, 1e-6)
    assert q.shape == (2, 8, 32) and k.shape == (2, 2, 32) and v.shape == (2, 2, 32) and slots.dtype == torch.int64
    out = ops.hif8_gdn_decode_step(
        torch.empty(2, 320, dtype=torch.bfloat16, **meta), torch.empty(2, 8, dtype=torch.bfloat16, **meta),
        torch.empty(320, 4, dtype=torch.bfloat16, **meta), torch.empty(2, 320, 3, dtype=torch.bfloat16, **meta),
        torch.empty(4, **meta), torch.empty(4, **meta), torch.empty(2, 4, 32, 48, **meta),
        torch.empty(48, dtype=torch.bfloat16, **meta), 2, 4, 32, 48, 1e-6)
    assert out.shape == (2, 4 * 48) and out.dtype == torch.bfloat16
    c3, r3 = ops.hif8_gate_up_silu_mul_quant(torch.empty(3, 64, dtype=torch.uint8, **meta),
                                             torch.empty(10, 64, dtype=torch.uint8, **meta), torch.empty(3, **meta),
                                             torch.empty(10, **meta), torch.empty(1, **meta))
    assert c3.shape == (3, 5) and c3.dtype == torch.uint8 and r3.shape == (3,)
    out = ops.hif8_gdn_decode_token(
        torch.empty(2, 320, dtype=torch.bfloat16, **meta), torch.empty(2, 64, dtype=torch.bfloat16, **meta),
        torch.empty(8, 64, dtype=torch.bfloat16, **meta), torch.empty(320, 4, dtype=torch.bfloat16, **meta),
        torch.empty(2, 320, 3, dtype=torch.bfloat16, **meta), torch.empty(4, **meta), torch.empty(4, **meta),
        torch.empty(2, 4, 32, 48, **meta), torch.empty(48, dtype=torch.bfloat16, **meta), 2, 4, 32, 48, 1e-6)
    assert out.shape == (2, 4 * 48) and out.dtype == torch.bfloat16
    y, conv = ops.hif8_linear_conv(torch.empty(2, 64, dtype=torch.uint8, **meta),
                                   torch.empty(512, 64, dtype=torch.uint8, **meta), torch.empty(2, **meta),
                                   torch.empty(512, **meta), torch.empty(320, 4, dtype=torch.bfloat16, **meta),
                                   torch.empty(2, 320, 3, dtype=torch.bfloat16, **meta))
    assert y.shape == (2, 512) and y.dtype == torch.bfloat16 and conv.shape == (2, 320) and conv.dtype == torch.float32
    out = ops.hif8_gdn_decode_head(
        torch.empty(2, 320, **meta), torch.empty(2, 512, dtype=torch.bfloat16, **meta),
        torch.empty(2, 64, dtype=torch.bfloat16, **meta), torch.empty(8, 64, dtype=torch.bfloat16, **meta),
        torch.empty(4, **meta), torch.empty(4, **meta), torch.empty(2, 4, 32, 48, **meta),
        torch.empty(48, dtype=torch.bfloat16, **meta), 2, 4, 32, 48, 1e-6)
    assert out.shape == (2, 4 * 48) and out.dtype == torch.bfloat16


def test_embedding_method_validates_weights_without_a_gpu(monkeypatch):
    from hif8_rocm import scheme

    layer = torch.nn.Module()
    layer.weight = torch.nn.Parameter(torch.zeros(4, 8), requires_grad=False)
    layer.weight_scale = torch.nn.Parameter(torch.ones(4, 1), requires_grad=False)
    method = scheme.W8A8HiFloat8SoftEmbeddingMethod()
    with pytest.raises(TypeError, match="torch.uint8"):
        method.process_weights_after_loading(layer)
    layer.weight = torch.nn.Parameter(torch.zeros(4, 8, dtype=torch.uint8), requires_grad=False)
    method.process_weights_after_loading(layer)
    assert layer.weight_scale.shape == (4,)
    monkeypatch.setenv("HIF8_COMPUTE_BACKEND", "other")
    with pytest.raises(ValueError, match="soft_hif8"):
        method.process_weights_after_loading(layer)


def test_offset_and_strided_views_are_materialized():
    base = torch.arange(24, dtype=torch.uint8).reshape(6, 4)
    for view in (base[2:], base[:, ::2]):
        out = native._as_native_operand(view)
        assert out.storage_offset() == 0 and out.is_contiguous() and torch.equal(out, view)
    clean = torch.zeros((3, 4), dtype=torch.uint8)
    assert native._as_native_operand(clean) is clean


def test_soft_linear_feeds_clean_operands_and_reshapes():
    seen = {}

    def fake_gemm(activation, weight, token_scale, channel_scale, bias, output_dtype):
        seen["offsets"] = [t.storage_offset() for t in (activation, token_scale, channel_scale)]
        seen["contig"] = [t.is_contiguous() for t in (activation, token_scale, channel_scale)]
        return torch.zeros((activation.shape[0], weight.shape[0]), dtype=output_dtype)

    ext = types.SimpleNamespace(hif8_static_quant=None, soft_hif8_gemv=fake_gemm, soft_hif8_gemm=fake_gemm)
    activation = torch.zeros((5, 2, 4), dtype=torch.uint8)[1:]
    scale = torch.ones(10, dtype=torch.float32)[2:]
    with patch.object(native, "load_extension", return_value=ext), \
         patch.object(native, "_operator", lambda name, e: getattr(e, name)):
        out = native.soft_linear(activation, torch.zeros((3, 4), dtype=torch.uint8), scale,
                                 torch.ones(3, dtype=torch.float32), None, output_dtype=torch.float32)
    assert seen["offsets"] == [0, 0, 0] and all(seen["contig"])
    assert tuple(out.shape) == (4, 2, 3)


def test_soft_linear_routes_like_the_reference():
    calls = []

    def op(kind):
        def f(activation, weight, *rest):
            calls.append(kind)
            return torch.zeros((activation.shape[0], weight.shape[0]), dtype=torch.bfloat16)
        return f

    ext = types.SimpleNamespace(soft_hif8_gemv=op("gemv"), soft_hif8_gemm=op("gemm"))
    s2 = torch.ones(2, dtype=torch.float32)
    with patch.object(native, "load_extension", return_value=ext), \
         patch.object(native, "_operator", lambda name, e: getattr(e, name)):
        for m, n, k in ((1, 3, 4), (2, 3, 4), (1, 1536, 4), (1, 1664, 4), (1, 512, 8192), (1, 512, 12288)):
            native.soft_linear(torch.zeros((m, k), dtype=torch.uint8), torch.zeros((n, k), dtype=torch.uint8),
                               s2[:m], torch.ones(n, dtype=torch.float32), output_dtype=torch.bfloat16)
        with patch.dict(os.environ, {"HIF8_DISABLE_GEMV": "1"}):
            native.soft_linear(torch.zeros((1, 4), dtype=torch.uint8), torch.zeros((3, 4), dtype=torch.uint8),
                               s2[:1], torch.ones(3, dtype=torch.float32), output_dtype=torch.bfloat16)
    assert calls == ["gemv", "gemm", "gemv", "gemm", "gemv", "gemm", "gemm"]


def test_static_quant_validation_messages():
    with pytest.raises(TypeError, match="FP16/BF16"):
        native.static_quant(torch.zeros(2, 4, dtype=torch.float32), torch.ones(1))
    with pytest.raises(TypeError, match="1D torch.float32"):
        native.static_quant(torch.zeros(2, 4, dtype=torch.bfloat16), torch.ones(1, dtype=torch.float64))
    with pytest.raises(ValueError, match="must divide"):
        native.static_quant(torch.zeros(3, 4, dtype=torch.bfloat16), torch.ones(2))


# --------------------------------------------------------------- scheme

def _layer(input_scale=0.25, k=8):
    layer = torch.nn.Module()
    layer.weight = torch.nn.Parameter(torch.zeros((5, k), dtype=torch.uint8), requires_grad=False)
    layer.weight_scale = torch.nn.Parameter(torch.ones((5, 1), dtype=torch.float32), requires_grad=False)
    layer.input_scale = torch.nn.Parameter(torch.tensor([input_scale], dtype=torch.float32), requires_grad=False)
    return layer


@pytest.fixture
def clean_env():
    with patch.dict(os.environ, {}, clear=False):
        for var in ("HIF8_COMPUTE_BACKEND", "HIF8_STATIC_FUSED_GENERATION", "HIF8_STATIC_SCALE_FACTOR",
                    "HIF8_STATIC_FUSED_SINGLE_ROW", "HIF8_STATIC_FUSED_ROWS", "HIF8_PREFILL_BF16_WEIGHTS"):
            os.environ.pop(var, None)
        yield


def test_declares_one_fp32_input_scale(clean_env):
    params = W8A8HiFloat8StaticLinearMethod().get_pertensor_param(torch.bfloat16, layer_type="others")
    assert set(params) == {"input_scale"}
    assert params["input_scale"].dtype == torch.float32 and tuple(params["input_scale"].shape) == (1,)
    assert STATIC_QUANT_TYPE == "W8A8HIF8_STATIC"


@pytest.mark.parametrize("value", [0.0, -1.0, float("inf"), float("nan")])
def test_rejects_invalid_input_scales(clean_env, value):
    with pytest.raises(ValueError, match="finite and greater"):
        W8A8HiFloat8StaticLinearMethod().process_weights_after_loading(_layer(value))


def test_rejects_non_scalar_input_scale(clean_env):
    layer = _layer()
    layer.input_scale = torch.nn.Parameter(torch.ones(2, dtype=torch.float32), requires_grad=False)
    with pytest.raises(ValueError, match="one input_scale"):
        W8A8HiFloat8StaticLinearMethod().process_weights_after_loading(layer)


def test_rejects_unsupported_backend(clean_env):
    os.environ["HIF8_COMPUTE_BACKEND"] = "unsupported"
    with pytest.raises(ValueError, match="unsupported"):
        W8A8HiFloat8StaticLinearMethod().process_weights_after_loading(_layer())


def test_apply_defaults_to_standalone_static_quant(clean_env):
    method = W8A8HiFloat8StaticLinearMethod()
    layer = _layer()
    method.process_weights_after_loading(layer)
    assert tuple(layer.weight_scale.shape) == (5,)
    x = torch.randn((5, 8), dtype=torch.bfloat16)  # more rows than the decode-sized fused route takes
    enc, rs, out = torch.zeros_like(x, dtype=torch.uint8), torch.full((5,), 0.25), torch.randn(5, 5)
    with patch("hif8_rocm.scheme.native.static_quant", return_value=(enc, rs)) as sq, \
         patch("hif8_rocm.scheme.native.soft_static_fused_linear") as fused, \
         patch("hif8_rocm.scheme.native.soft_linear", return_value=out) as lin:
        assert method.apply(layer, x, None) is out
    sq.assert_called_once_with(x, layer.input_scale)
    fused.assert_not_called()
    lin.assert_called_once_with(enc, layer.weight, rs, layer.weight_scale, None, output_dtype=x.dtype)


def test_fused_generation_is_opt_in_and_limited_to_small_shapes(clean_env):
    # The reference's routing contract (test_static_scheme.py:105-192), which
    # HIF8_STATIC_FUSED_SINGLE_ROW=0 restores for one-row inputs too.
    os.environ["HIF8_STATIC_FUSED_SINGLE_ROW"] = "0"
    os.environ["HIF8_STATIC_FUSED_GENERATION"] = "1"
    method = W8A8HiFloat8StaticLinearMethod()
    layer = _layer()
    method.process_weights_after_loading(layer)
    out = torch.randn(2, 5)
    with patch("hif8_rocm.scheme.native.static_quant") as sq, \
         patch("hif8_rocm.scheme.native.soft_linear") as lin, \
         patch("hif8_rocm.scheme.native.soft_static_fused_linear", return_value=out) as fused:
        assert method.apply(layer, torch.randn((2, 8), dtype=torch.bfloat16)) is out
    sq.assert_not_called()
    lin.assert_not_called()
    fused.assert_called_once()
    # M = 5 and model-sized K keep the two-stage path.
    for shape, k in (((5, 8), 8), ((1, 4096), 4096)):
        layer = _layer(k=k)
        method.process_weights_after_loading(layer)
        x = torch.zeros(shape, dtype=torch.bfloat16)
        with patch("hif8_rocm.scheme.native.static_quant", return_value=(x.to(torch.uint8), torch.ones(shape[0]))) as sq, \
             patch("hif8_rocm.scheme.native.soft_linear", return_value=out), \
             patch("hif8_rocm.scheme.native.soft_static_fused_linear") as fused:
            method.apply(layer, x)
        sq.assert_called_once()
        fused.assert_not_called()


def test_decode_row_fusion_is_the_default_with_an_opt_out(clean_env):
    """Up to four token rows go through the fused op by default, whatever K,
    and nothing larger does; HIF8_STATIC_FUSED_SINGLE_ROW=0 or
    HIF8_STATIC_FUSED_ROWS=0 restores the reference's two-stage routing and
    HIF8_STATIC_FUSED_ROWS=1 fuses one row only."""
    method = W8A8HiFloat8StaticLinearMethod()
    out = torch.randn(1, 5)
    cases = [(None, None, (1, 4096), True), ("1", None, (1, 4096), True), ("0", None, (1, 4096), False),
             (None, None, (1, 8), True), (None, None, (2, 4096), True), ("1", None, (3, 64), True),
             (None, None, (4, 4096), True), (None, None, (5, 4096), False), (None, None, (1, 12288), True),
             ("0", None, (1, 12288), False), ("0", None, (1, 64), False), ("0", "4", (4, 64), False),
             (None, "0", (1, 4096), False), (None, "1", (1, 4096), True), (None, "1", (2, 4096), False),
             (None, "3", (3, 4096), True), (None, "3", (4, 4096), False), (None, "9", (4, 64), True)]
    for flag, rows_env, shape, want_fused in cases:
        for var, val in (("HIF8_STATIC_FUSED_SINGLE_ROW", flag), ("HIF8_STATIC_FUSED_ROWS", rows_env)):
            if val is None:
                os.environ.pop(var, None)
            else:
                os.environ[var] = val
        layer = _layer(k=shape[1])
        method.process_weights_after_loading(layer)
        x = torch.zeros(shape, dtype=torch.bfloat16)
        with patch("hif8_rocm.scheme.native.static_quant",
                   return_value=(x.to(torch.uint8), torch.ones(shape[0]))) as sq, \
             patch("hif8_rocm.scheme.native.soft_linear", return_value=out), \
             patch("hif8_rocm.scheme.native.soft_static_fused_linear", return_value=out) as fused:
            method.apply(layer, x)
        assert fused.called == want_fused and sq.called != want_fused, (flag, rows_env, shape)
        if want_fused:
            fused.assert_called_once_with(x, layer.weight, layer.input_scale, layer.weight_scale, None,
                                          output_dtype=x.dtype)


def test_prefill_bf16_weights_route_only_large_m(clean_env):
    """A layer holding a decoded weight runs M > 4 on it; M <= 4 keeps the codes
    (two-stage routing, so that one row is not fused)."""
    os.environ["HIF8_STATIC_FUSED_SINGLE_ROW"] = "0"
    method = W8A8HiFloat8StaticLinearMethod()
    layer = _layer(k=64)
    method.process_weights_after_loading(layer)
    assert layer._hif8_weight_bf16 is None  # opt-in only (and CPU tensors are never decoded)
    layer._hif8_weight_bf16 = torch.zeros(5, 64, dtype=torch.bfloat16)
    for rows, want_decoded in ((5, True), (512, True), (4, False), (1, False)):
        x = torch.zeros((rows, 64), dtype=torch.bfloat16)
        enc, rs = x.to(torch.uint8), torch.ones(rows)
        with patch("hif8_rocm.scheme.native.static_quant", return_value=(enc, rs)), \
             patch("hif8_rocm.scheme.native.soft_linear") as lin, \
             patch("hif8_rocm.scheme.native.soft_linear_decoded_weight") as dec:
            method.apply(layer, x)
        assert dec.called == want_decoded and lin.called != want_decoded, rows
        if want_decoded:
            dec.assert_called_once_with(enc, layer._hif8_weight_bf16, rs, layer.weight_scale, None,
                                        output_dtype=x.dtype)


def test_decoded_weight_wrappers_validate_dtypes():
    with pytest.raises(TypeError, match="uint8"):
        native.decode_weight(torch.zeros(4, 16, dtype=torch.float32))
    with pytest.raises(ValueError, match="multiple of 16"):
        native.decode_weight(torch.zeros(3, 5, dtype=torch.uint8))
    with pytest.raises(TypeError, match="bfloat16 weight"):
        native.soft_linear_decoded_weight(torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(4, 64, dtype=torch.uint8),
                                          torch.ones(8), torch.ones(4), output_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="incompatible K"):
        native.soft_linear_decoded_weight(torch.zeros(8, 64, dtype=torch.uint8),
                                          torch.zeros(4, 128, dtype=torch.bfloat16), torch.ones(8), torch.ones(4),
                                          output_dtype=torch.bfloat16)


def test_scale_factor_env_multiplies_the_checkpoint_scale(clean_env):
    os.environ["HIF8_STATIC_SCALE_FACTOR"] = "2.0"
    method = W8A8HiFloat8StaticLinearMethod()
    layer = _layer(0.25)
    method.process_weights_after_loading(layer)
    x = torch.zeros((6, 8), dtype=torch.bfloat16)
    with patch("hif8_rocm.scheme.native.static_quant", return_value=(x.to(torch.uint8), torch.ones(6))) as sq, \
         patch("hif8_rocm.scheme.native.soft_linear", return_value=torch.zeros(6, 5)):
        method.apply(layer, x)
    assert float(sq.call_args[0][1]) == 0.5
    # Decode-sized inputs take the fused op, with the same scaled fixed scale.
    with patch("hif8_rocm.scheme.native.soft_static_fused_linear", return_value=torch.zeros(1, 5)) as fused:
        method.apply(layer, x[:1])
    assert float(fused.call_args[0][2]) == 0.5
    os.environ["HIF8_STATIC_SCALE_FACTOR"] = "-1"
    with pytest.raises(ValueError, match="positive finite"):
        method.apply(layer, x)


def test_soft_method_defaults_to_dynamic_quant_then_soft_linear(clean_env):
    from hif8_rocm.scheme import SOFT_QUANT_TYPE, W8A8HiFloat8SoftLinearMethod

    os.environ.pop("HIF8_SOFT_FUSED_GENERATION", None)
    method = W8A8HiFloat8SoftLinearMethod()
    assert method.quant_type == SOFT_QUANT_TYPE == "W8A8HIF8_SOFT"
    layer = _layer()
    del layer.input_scale
    method.process_weights_after_loading(layer)
    x = torch.randn((2, 8), dtype=torch.bfloat16)
    enc, ts, out = torch.zeros_like(x, dtype=torch.uint8), torch.full((2,), 3.0), torch.randn(2, 5)
    with patch("hif8_rocm.scheme.native.dynamic_quant", return_value=(enc, ts)) as dq, \
         patch("hif8_rocm.scheme.native.soft_fused_linear") as fused, \
         patch("hif8_rocm.scheme.native.soft_linear", return_value=out) as lin:
        assert method.apply(layer, x, None) is out
    dq.assert_called_once_with(x)
    fused.assert_not_called()
    lin.assert_called_once_with(enc, layer.weight, ts, layer.weight_scale, None, output_dtype=x.dtype)


def test_soft_fused_generation_is_opt_in_for_two_rows(clean_env):
    from hif8_rocm.scheme import W8A8HiFloat8SoftLinearMethod

    os.environ["HIF8_SOFT_FUSED_GENERATION"] = "1"
    try:
        method = W8A8HiFloat8SoftLinearMethod()
        layer = _layer()
        method.process_weights_after_loading(layer)
        out = torch.randn(2, 5)
        with patch("hif8_rocm.scheme.native.dynamic_quant") as dq, \
             patch("hif8_rocm.scheme.native.soft_fused_linear", return_value=out) as fused:
            assert method.apply(layer, torch.randn((2, 8), dtype=torch.bfloat16)) is out
        dq.assert_not_called()
        fused.assert_called_once()
        x = torch.zeros((3, 8), dtype=torch.bfloat16)
        with patch("hif8_rocm.scheme.native.dynamic_quant", return_value=(x.to(torch.uint8), torch.ones(3))) as dq, \
             patch("hif8_rocm.scheme.native.soft_linear", return_value=out), \
             patch("hif8_rocm.scheme.native.soft_fused_linear") as fused:
            method.apply(layer, x)
        dq.assert_called_once()
        fused.assert_not_called()
    finally:
        os.environ.pop("HIF8_SOFT_FUSED_GENERATION", None)


def test_soft_fused_linear_validates_like_the_reference():
    w = torch.zeros(4, 8, dtype=torch.uint8)
    with pytest.raises(TypeError, match="FP16/BF16 activation"):
        native.soft_fused_linear(torch.zeros(1, 8), w, torch.ones(4), output_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="compatible final K"):
        native.soft_fused_linear(torch.zeros(1, 7, dtype=torch.bfloat16), w, torch.ones(4), output_dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="one float32 scale per output channel"):
        native.soft_fused_linear(torch.zeros(1, 8, dtype=torch.bfloat16), w, torch.ones(3), output_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="M <= 2"):
        native.soft_fused_linear(torch.zeros(3, 8, dtype=torch.bfloat16), w, torch.ones(4), output_dtype=torch.bfloat16)
