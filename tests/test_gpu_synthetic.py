"""The synthetic hybrid model (config-5 workload) on the GPU at a tiny size:
decode steps (GEMV, fused KV write, paged HiF8 attention, recurrent gated
delta rule) agree with a prefill of the same tokens (GEMM, attention over
decoded cache rows, chunked delta rule), and graph replay reproduces eager
decoding token for token."""

import pytest
import torch

pytestmark = pytest.mark.gpu

TINY = dict(hidden=256, layers=4, heads=4, kv_heads=2, head_dim=64, rotary_dim=16, intermediate=512,
            lin_k_heads=2, lin_v_heads=4, lin_k_dim=32, lin_v_dim=32, vocab=1000, block_size=16)


@pytest.fixture(scope="module")
def model(native_ops, device):
    from hif8_rocm.synthetic_model import HybridConfig, HybridModel

    m = HybridModel(HybridConfig(**TINY), device, seed=0)
    m.calibrate(batch=1, tokens=32)
    return m


def test_calibration_sets_finite_scales(model):
    from hif8_rocm.synthetic_model import StaticLinear

    for L in model.layers:
        for v in L.values():
            if isinstance(v, StaticLinear):
                s = float(v.layer.input_scale)
                assert s > 0 and s == s and s != float("inf")
        if "k_scale" in L:
            assert bool((L["k_scale"] > 0).all()) and bool((L["v_scale"] > 0).all())


def test_decode_steps_agree_with_prefill(model, device):
    b, t, steps = 2, 20, 4
    g = torch.Generator(device=device).manual_seed(3)
    prompt = torch.randint(0, model.cfg.vocab, (b, t), generator=g, device=device)
    st = model.new_state(b, t + steps + 1)
    pos = torch.arange(t, device=device).expand(b, t).contiguous()
    st.seq_lens.fill_(t)
    logits = model.forward(st, prompt, pos, decode=False)
    toks = [logits.argmax(-1, keepdim=True)]
    for j in range(steps):
        st.seq_lens.add_(1)
        logits = model.forward(st, toks[-1], torch.full((b, 1), t + j, device=device), decode=True)
        toks.append(logits.argmax(-1, keepdim=True))
    assert bool(torch.isfinite(logits).all())
    full = torch.cat([prompt] + toks[:steps], dim=1)
    st2 = model.new_state(b, full.shape[1])
    pos2 = torch.arange(full.shape[1], device=device).expand(b, -1).contiguous()
    st2.seq_lens.fill_(full.shape[1])
    ref = model.forward(st2, full, pos2, decode=False)
    cos = torch.nn.functional.cosine_similarity(logits, ref, dim=-1)
    assert float(cos.min()) > 0.995, cos


def test_prefill_rejects_stale_sequence_lengths(model, device):
    # seq_lens must cover the prefill's rows (last position + 1); a stale value
    # would make rows see no keys, so the forward refuses it.
    st = model.new_state(2, 16)
    ids = torch.zeros(2, 8, dtype=torch.int64, device=device)
    pos = torch.arange(8, device=device).expand(2, 8).contiguous()
    with pytest.raises(ValueError, match="seq_lens"):
        model.forward(st, ids, pos, decode=False)
    st.seq_lens.fill_(8)
    assert bool(torch.isfinite(model.forward(st, ids, pos, decode=False)).all())


def test_chunked_prefill_continues_the_cached_request(model, device):
    """A prompt prefilled in two chunks (the second chunk's rows attend the
    first chunk's cached pages through the right-aligned causal mask, and the
    linear-attention layers carry their conv / recurrent state) gives the
    logits of one prefill of the whole prompt."""
    b, t1, t2 = 2, 20, 13
    g = torch.Generator(device=device).manual_seed(4)
    prompt = torch.randint(0, model.cfg.vocab, (b, t1 + t2), generator=g, device=device)
    whole = model.new_state(b, t1 + t2)
    whole.seq_lens.fill_(t1 + t2)
    ref = model.forward(whole, prompt, torch.arange(t1 + t2, device=device).expand(b, -1).contiguous(), decode=False)
    st = model.new_state(b, t1 + t2)
    st.seq_lens.fill_(t1)
    model.forward(st, prompt[:, :t1], torch.arange(t1, device=device).expand(b, -1).contiguous(), decode=False)
    st.seq_lens.fill_(t1 + t2)
    got = model.forward(st, prompt[:, t1:], torch.arange(t1, t1 + t2, device=device).expand(b, -1).contiguous(),
                        decode=False)
    cos = torch.nn.functional.cosine_similarity(got, ref, dim=-1)
    assert float(cos.min()) > 0.995, cos
    assert torch.equal(got.argmax(-1), ref.argmax(-1))


def test_graph_replay_matches_eager_decode(model, device):
    from hif8_rocm.synthetic_model import generate

    g = torch.Generator(device=device).manual_seed(5)
    prompt = torch.randint(0, model.cfg.vocab, (2, 24), generator=g, device=device)
    eager, _ = generate(model, prompt, 8, graph=False)
    graphed, timings = generate(model, prompt, 8, graph=True)
    assert torch.equal(eager, graphed)
    assert timings["prefill"] > 0 and timings["decode"] > 0 and timings["decode_steps"] == 6


def test_single_row_fusion_generates_the_same_tokens(model, device, monkeypatch):
    """One-row projections through the fused kernel (the default) and through
    quant -> GEMV (HIF8_STATIC_FUSED_SINGLE_ROW=0) give the same logits,
    hence the same tokens.  The
    glue-kernel input quant is switched off, so that every one-row projection
    (qkv / qkvz, gate_up, o / out, down) goes through the scheme and the fused
    op, not only the o / out projections."""
    from hif8_rocm.synthetic_model import generate

    g = torch.Generator(device=device).manual_seed(21)
    prompt = torch.randint(0, model.cfg.vocab, (1, 12), generator=g, device=device)
    monkeypatch.setenv("HIF8_STATIC_FUSED_SINGLE_ROW", "0")
    glue, _ = generate(model, prompt, 6, graph=True)
    monkeypatch.setattr(model, "fuse_input_quant", False)
    plain, _ = generate(model, prompt, 6, graph=True)
    monkeypatch.delenv("HIF8_STATIC_FUSED_SINGLE_ROW", raising=False)
    fused, _ = generate(model, prompt, 6, graph=True)
    assert torch.equal(plain, fused)
    assert torch.equal(glue, plain)


def test_fused_input_quant_generates_the_same_tokens(model, device):
    """Decode with the projections' input quant inside the norm and SiLU-mul
    kernels (the default) and with the scheme's own quant per projection:
    the codes are equal, so the tokens are too."""
    from hif8_rocm.synthetic_model import generate

    assert model._fuse_input_quant()
    g = torch.Generator(device=device).manual_seed(23)
    prompt = torch.randint(0, model.cfg.vocab, (2, 12), generator=g, device=device)
    fused, _ = generate(model, prompt, 6, graph=True)
    model.fuse_input_quant = False
    try:
        plain, _ = generate(model, prompt, 6, graph=True)
    finally:
        model.fuse_input_quant = True
    assert torch.equal(plain, fused)


@pytest.mark.parametrize("rows,n", [(1, 4096), (4, 4096), (3, 8)])
def test_glue_with_input_quant_equals_glue_then_static_quant(native_ops, device, rows, n):
    """hif8_add_rms_norm_quant and hif8_silu_mul_quant: the bf16 result of the
    plain glue op and, bit for bit, the codes and row scales that
    hif8_static_quant gives for it (scales from fine to saturating, NaN and
    Inf inputs)."""
    from hif8_rocm import native

    ops = torch.ops.vllm_ascend_hif8
    g = torch.Generator(device=device).manual_seed(rows * 1000 + n)
    h = (torch.randn(rows, n, generator=g, device=device) * 3).to(torch.bfloat16)
    d = torch.randn(rows, n, generator=g, device=device).to(torch.bfloat16)
    w = (torch.rand(n, generator=g, device=device) + 0.5).to(torch.bfloat16)
    gu = (torch.randn(rows, 2 * n, generator=g, device=device) * 2).to(torch.bfloat16)
    gu[0, 5] = float("nan")
    gu[-1, n + 6] = float("inf")
    for sv in (1e-6, 1e-3, 0.037, 1.0):
        s = torch.tensor([sv], dtype=torch.float32, device=device)
        for delta in (d, None):
            want_h = h.clone()
            want = ops.hif8_add_rms_norm(want_h, delta, w, 1e-6)
            got_h = h.clone()
            got, codes, rs = ops.hif8_add_rms_norm_quant(got_h, delta, w, 1e-6, s)
            assert torch.equal(got_h, want_h) and torch.equal(got, want)
            want_codes, want_rs = native.static_quant(want, s)
            assert torch.equal(codes, want_codes), (sv, delta is None)
            assert torch.equal(rs.reshape(-1), want_rs.reshape(-1))
        codes, rs = ops.hif8_silu_mul_quant(gu, s)
        want_codes, want_rs = native.static_quant(ops.hif8_silu_mul(gu), s)
        assert torch.equal(codes, want_codes), sv
        assert torch.equal(rs.reshape(-1), want_rs.reshape(-1))
    assert codes[0, 5].item() == 0x80  # NaN


def test_fused_add_rms_norm_silu_mul_and_bf16_gemv_match_torch(native_ops, device):
    from hif8_rocm.synthetic_model import rms_norm

    g = torch.Generator(device=device).manual_seed(7)
    h = torch.randn(3, 4096, generator=g, device=device).to(torch.bfloat16)
    d = torch.randn(3, 4096, generator=g, device=device).to(torch.bfloat16)
    w = (torch.rand(4096, generator=g, device=device) + 0.5).to(torch.bfloat16)
    want_h = h + d
    want = rms_norm(want_h, w, 1e-6)
    got_h = h.clone()
    got = torch.ops.vllm_ascend_hif8.hif8_add_rms_norm(got_h, d, w, 1e-6)
    assert torch.equal(got_h, want_h)
    torch.testing.assert_close(got.float(), want.float(), rtol=1e-2, atol=1e-2)
    plain = torch.ops.vllm_ascend_hif8.hif8_add_rms_norm(h.clone(), None, w, 1e-6)
    torch.testing.assert_close(plain.float(), rms_norm(h, w, 1e-6).float(), rtol=1e-2, atol=1e-2)
    # a width the 16-byte path does not take (n % 8 != 0): the scalar kernel
    h3 = torch.randn(2, 1004, generator=g, device=device).to(torch.bfloat16)
    d3 = torch.randn(2, 1004, generator=g, device=device).to(torch.bfloat16)
    w3 = (torch.rand(1004, generator=g, device=device) + 0.5).to(torch.bfloat16)
    got3_h = h3.clone()
    got3 = torch.ops.vllm_ascend_hif8.hif8_add_rms_norm(got3_h, d3, w3, 1e-6)
    assert torch.equal(got3_h, h3 + d3)
    torch.testing.assert_close(got3.float(), rms_norm(h3 + d3, w3, 1e-6).float(), rtol=1e-2, atol=1e-2)
    for m, n, k in ((1, 64, 4096), (3, 37, 264), (4, 8, 8)):
        x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
        w = torch.randn(n, k, generator=g, device=device).to(torch.bfloat16)
        y = torch.ops.vllm_ascend_hif8.hif8_bf16_gemv(x, w)
        torch.testing.assert_close(y.float(), (x.float() @ w.float().t()), rtol=1e-2, atol=1e-2)
    gu = torch.randn(5, 600, generator=g, device=device).to(torch.bfloat16)
    act = torch.ops.vllm_ascend_hif8.hif8_silu_mul(gu)
    ref = (torch.nn.functional.silu(gu[:, :300].float()) * gu[:, 300:].float()).to(torch.bfloat16)
    torch.testing.assert_close(act.float(), ref.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m,inter,k", [(1, 12288, 4096), (2, 12288, 4096), (4, 12288, 4096), (1, 37, 64),
                                       (3, 500, 256), (1, 2048, 12288)])
def test_fused_gate_up_silu_mul_quant_equals_gemv_then_silu_mul_quant(m, inter, k, native_ops, device):
    """hif8_gate_up_silu_mul_quant: the gate_up GEMV whose blocks pair gate
    and up rows and finish with SiLU-mul and the static quant gives the codes
    of soft_hif8_gemm (bf16) + SiLU-mul + static quant bit for bit (where the
    GEMV plan is not the dot2 kernel, e.g. M = 4 over wide weights, the op
    runs soft_hif8_gemm + hif8_silu_mul_quant itself)."""
    ops = torch.ops.vllm_ascend_hif8
    g = torch.Generator(device=device).manual_seed(m * 7 + inter + k)
    w = torch.randn(2 * inter, k, generator=g, device=device).to(torch.bfloat16)
    from hif8_rocm import native
    ws = (w.float().abs().amax(dim=1) / 32768.0).contiguous()
    wq, _ = native.static_quant(w, ws)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    xs = (x.float().abs().amax() / 32768.0).reshape(1)
    a, rs = native.static_quant(x, xs)
    a[0, :3] = torch.tensor([0x80, 0x6F, 0xEF], dtype=torch.uint8, device=device)  # NaN, +Inf, -Inf codes
    for sv in (1e-6, 0.01, 3.0):
        s = torch.tensor([sv], device=device)
        codes, out_rs = ops.hif8_gate_up_silu_mul_quant(a, wq, rs, ws, s)
        gu = ops.soft_hif8_gemm(a, wq, rs, ws, None, torch.bfloat16)
        # hif8_silu_mul_quant takes widths % 8 == 0 only; its codes equal these
        want, want_rs = native.static_quant(ops.hif8_silu_mul(gu), s)
        assert torch.equal(codes, want), (m, inter, k, sv)
        assert torch.equal(out_rs, want_rs.reshape(-1))


@pytest.mark.parametrize("shape", [
    # batch, k_heads, v_heads, k_dim, v_dim, hidden, conv width
    (1, 16, 32, 128, 128, 4096, 4),  # the full-size model
    (4, 16, 32, 128, 128, 4096, 4),
    (3, 2, 4, 32, 32, 256, 4),       # the tiny model
    (2, 3, 3, 64, 96, 520, 3),       # one value head per key head
    (2, 2, 6, 32, 32, 256, 4),       # three per key head: the two-launch fallback
])
def test_fused_decode_token_equals_bf16_gemv_plus_decode_step(shape, native_ops, device):
    """hif8_gdn_decode_token folds the b/a projection and the conv into the
    delta-rule kernel.  Against hif8_bf16_gemv + hif8_gdn_decode_step, step
    after step: the conv state is equal bit for bit (the same conv), the
    recurrent state agrees to FP32 rounding (the fused kernel scales the
    state dot products by 1/|k| and 1/(|q| sqrt(dk)) after the sum, the
    step kernel normalises q and k first), the bf16 outputs to one bf16
    step, and nearly all of them are equal."""
    b, kh, vh, dk, dv, hidden, kw = shape
    ops = torch.ops.vllm_ascend_hif8
    g = torch.Generator(device=device).manual_seed(sum(shape))
    channels = 2 * kh * dk + vh * dv
    bf = torch.bfloat16
    ba_w = (torch.randn(2 * vh, hidden, generator=g, device=device) * 0.05).to(bf)
    conv_w = (torch.randn(channels, kw, generator=g, device=device) * 0.5).to(bf)
    a_log = torch.randn(vh, generator=g, device=device) * 0.5
    dt_bias = torch.randn(vh, generator=g, device=device) * 0.5
    out_norm = (torch.rand(dv, generator=g, device=device) + 0.5).to(bf)
    conv_a = torch.randn(b, channels, kw - 1, generator=g, device=device).to(bf)
    rec_a = torch.randn(b, vh, dk, dv, generator=g, device=device) * 0.1
    conv_b, rec_b = conv_a.clone(), rec_a.clone()
    for step in range(3):
        mixed = torch.randn(b, channels + vh * dv, generator=g, device=device).to(bf)
        x = torch.randn(b, hidden, generator=g, device=device).to(bf)
        got = ops.hif8_gdn_decode_token(mixed, x, ba_w, conv_w, conv_a, a_log, dt_bias, rec_a, out_norm,
                                        kh, vh, dk, dv, 1e-6)
        want = ops.hif8_gdn_decode_step(mixed, ops.hif8_bf16_gemv(x, ba_w), conv_w, conv_b, a_log, dt_bias, rec_b,
                                        out_norm, kh, vh, dk, dv, 1e-6)
        assert torch.equal(conv_a, conv_b), (shape, step)
        torch.testing.assert_close(rec_a, rec_b, rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(got.float(), want.float(), rtol=8e-3, atol=1e-5)
        assert (got == want).float().mean().item() > 0.9, (shape, step)


def _conv_reference(y, state, w):
    """Float32 causal conv + SiLU of the first channels of y [m, n] (bf16)
    over state [m, channels, kw - 1], taps in order (hif8_gdn_decode_step's
    conv); returns the outputs and the shifted state."""
    channels, kw = w.shape
    x = y[:, :channels]
    acc = torch.zeros(x.shape, dtype=torch.float32, device=x.device)
    for t in range(kw - 1):
        acc = acc + state[:, :, t].float() * w[:, t].float()
    acc = acc + x.float() * w[:, kw - 1].float()
    shifted = torch.cat([state[:, :, 1:], x[:, :, None]], dim=2)
    return acc / (1 + torch.exp(-acc)), shifted


@pytest.mark.parametrize("shape", [
    # m, n, k, channels, conv width
    (1, 12288, 4096, 8192, 4),  # the full-size qkvz projection: dot2 GEMV epilogue
    (4, 12288, 4096, 8192, 4),  # MFMA-4 GEMV epilogue
    (2, 640, 256, 384, 3),
    (3, 200, 64, 100, 2),
    (1, 96, 40, 96, 4),         # k % 16 != 0: the GEMV plan without the epilogue, then the conv kernel
    (6, 300, 128, 128, 4),      # m > 4: the GEMM, then the conv kernel
])
def test_linear_conv_equals_gemm_then_conv(shape, native_ops, device):
    """hif8_linear_conv: the bf16 projection equals soft_hif8_gemm bit for
    bit, the conv state shifts to the float32 reference's bit for bit, and
    the conv outputs agree with the float32 reference (the kernels contract
    the tap products into FMAs)."""
    from hif8_rocm import native

    m, n, k, channels, kw = shape
    ops = torch.ops.vllm_ascend_hif8
    g = torch.Generator(device=device).manual_seed(sum(shape))
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    a, rs = native.static_quant(x, torch.tensor([x.float().abs().max().item() / 12], device=device))
    w = torch.randn(n, k, generator=g, device=device).to(torch.bfloat16)
    wq, ws = native.static_quant(w, torch.tensor([w.float().abs().max().item()], device=device))
    ws = (ws.reshape(-1) * (torch.rand(n, generator=g, device=device) + 0.5)).contiguous()
    conv_w = (torch.randn(channels, kw, generator=g, device=device) * 0.5).to(torch.bfloat16)
    state = torch.randn(m, channels, kw - 1, generator=g, device=device).to(torch.bfloat16)
    for step in range(2):
        want_y = ops.soft_hif8_gemm(a, wq, rs, ws, None, torch.bfloat16)
        want_conv, want_state = _conv_reference(want_y, state, conv_w)
        y, conv = ops.hif8_linear_conv(a, wq, rs, ws, conv_w, state)
        assert torch.equal(y, want_y), (shape, step)
        assert torch.equal(state, want_state), (shape, step)
        torch.testing.assert_close(conv, want_conv, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("shape", [
    # batch, k_heads, v_heads, k_dim, v_dim, hidden, conv width
    (1, 16, 32, 128, 128, 4096, 4),  # the full-size model
    (4, 16, 32, 128, 128, 4096, 4),
    (3, 2, 4, 32, 32, 256, 4),       # the tiny model
    (2, 3, 3, 64, 96, 520, 3),       # one value head per key head
    (2, 2, 6, 32, 32, 256, 2),       # three per key head
])
def test_conv_gemv_plus_decode_head_equals_fused_token(shape, native_ops, device):
    """hif8_linear_conv + hif8_gdn_decode_head (the conv in the qkvz GEMV,
    one block per value head) against soft_hif8_gemm + hif8_gdn_decode_token
    (the conv in the per-group kernel), step after step: the projection and
    conv state bit for bit, the recurrent state to FP32 rounding, the bf16
    outputs to one bf16 step with nearly all equal."""
    from hif8_rocm import native

    b, kh, vh, dk, dv, hidden, kw = shape
    ops = torch.ops.vllm_ascend_hif8
    g = torch.Generator(device=device).manual_seed(sum(shape) + 1)
    channels = 2 * kh * dk + vh * dv
    n = channels + vh * dv
    bf = torch.bfloat16
    w = torch.randn(n, hidden, generator=g, device=device).to(bf)
    wq, ws = native.static_quant(w, torch.tensor([w.float().abs().max().item()], device=device))
    ws = (ws.reshape(-1) * (torch.rand(n, generator=g, device=device) * 0.05 + 0.01)).contiguous()
    ba_w = (torch.randn(2 * vh, hidden, generator=g, device=device) * 0.05).to(bf)
    conv_w = (torch.randn(channels, kw, generator=g, device=device) * 0.5).to(bf)
    a_log = torch.randn(vh, generator=g, device=device) * 0.5
    dt_bias = torch.randn(vh, generator=g, device=device) * 0.5
    out_norm = (torch.rand(dv, generator=g, device=device) + 0.5).to(bf)
    conv_a = torch.randn(b, channels, kw - 1, generator=g, device=device).to(bf)
    rec_a = torch.randn(b, vh, dk, dv, generator=g, device=device) * 0.1
    conv_b, rec_b = conv_a.clone(), rec_a.clone()
    for step in range(3):
        x = torch.randn(b, hidden, generator=g, device=device).to(bf)
        a, rs = native.static_quant(x, torch.tensor([x.float().abs().max().item() / 12], device=device))
        qkvz, conv = ops.hif8_linear_conv(a, wq, rs, ws, conv_w, conv_a)
        got = ops.hif8_gdn_decode_head(conv, qkvz, x, ba_w, a_log, dt_bias, rec_a, out_norm, kh, vh, dk, dv, 1e-6)
        mixed = ops.soft_hif8_gemm(a, wq, rs, ws, None, bf)
        want = ops.hif8_gdn_decode_token(mixed, x, ba_w, conv_w, conv_b, a_log, dt_bias, rec_b, out_norm,
                                         kh, vh, dk, dv, 1e-6)
        assert torch.equal(qkvz, mixed), (shape, step)
        assert torch.equal(conv_a, conv_b), (shape, step)
        torch.testing.assert_close(rec_a, rec_b, rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(got.float(), want.float(), rtol=8e-3, atol=1e-5)
        assert (got == want).float().mean().item() > 0.9, (shape, step)


def test_decode_head_rejects_unsupported_head_sizes(native_ops, device):
    ops = torch.ops.vllm_ascend_hif8
    bf = torch.bfloat16
    b, kh, vh, dk, dv, hidden = 1, 1, 1, 48, 32, 64
    channels = 2 * kh * dk + vh * dv
    conv = torch.zeros(b, channels, device=device)
    mixed = torch.zeros(b, channels + vh * dv, device=device, dtype=bf)
    x = torch.zeros(b, hidden, device=device, dtype=bf)
    with pytest.raises(RuntimeError, match="k_dim in"):
        ops.hif8_gdn_decode_head(conv, mixed, x, torch.zeros(2 * vh, hidden, device=device, dtype=bf),
                                 torch.zeros(vh, device=device), torch.zeros(vh, device=device),
                                 torch.zeros(b, vh, dk, dv, device=device), torch.ones(dv, device=device, dtype=bf),
                                 kh, vh, dk, dv, 1e-6)


@pytest.fixture(scope="module")
def odd_model(native_ops, device):
    """Linear-attention head sizes the wide delta-rule kernel does not take
    (k_dim % 8 != 0), so the fused step runs its general kernel."""
    from hif8_rocm.synthetic_model import HybridConfig, HybridModel

    cfg = dict(TINY, layers=2, lin_k_dim=20, lin_v_dim=24)
    return HybridModel(HybridConfig(**cfg), device, seed=1)


@pytest.mark.parametrize("which", ["model", "odd_model"])
@pytest.mark.parametrize("codes_in", [False, True])
def test_fused_linear_attention_step_matches_torch_step(which, codes_in, request, device):
    """The decode mixer against the torch step: from bf16 x (the per-group
    fused kernel) and from x's codes (the conv-epilogue GEMV + per-head
    kernel where the head sizes allow, as the decode step runs it)."""
    import copy

    from hif8_rocm import native

    model = request.getfixturevalue(which)
    c = model.cfg
    idx = 0
    L = model.layers[0]
    assert not c.is_full_attention(0)
    b = 3
    st_a = model.new_state(b, 8)
    g = torch.Generator(device=device).manual_seed(11)
    st_a.conv_states[idx].copy_(torch.randn(st_a.conv_states[idx].shape, generator=g, device=device))
    st_a.rec_states[idx].copy_(torch.randn(st_a.rec_states[idx].shape, generator=g, device=device) * 0.1)
    st_b = copy.copy(st_a)
    st_b.conv_states = [t.clone() for t in st_a.conv_states]
    st_b.rec_states = [t.clone() for t in st_a.rec_states]
    for step in range(3):
        x = torch.randn(b, c.hidden, generator=g, device=device).to(torch.bfloat16)
        xq = native.static_quant(x, L["qkvz"].layer.input_scale) if codes_in else None
        fused = model._linear_attention_decode(L, idx, st_a, x, xq)
        ref = model._linear_attention(L, idx, st_b, x[:, None], decode=True)[:, 0]
        torch.testing.assert_close(fused.float(), ref.float(), rtol=2e-2, atol=2e-2)
        torch.testing.assert_close(st_a.conv_states[idx], st_b.conv_states[idx])
        torch.testing.assert_close(st_a.rec_states[idx], st_b.rec_states[idx], rtol=1e-4, atol=1e-5)


def test_fused_attention_step_matches_torch_step(model, device):
    import copy

    c = model.cfg
    L = model.layers[3]
    assert c.is_full_attention(3)
    b, t = 2, 5
    g = torch.Generator(device=device).manual_seed(13)
    st_a = model.new_state(b, 40)
    st_b = copy.copy(st_a)
    st_b.key_caches = [kc.clone() for kc in st_a.key_caches]
    st_b.value_caches = [vc.clone() for vc in st_a.value_caches]
    for step in range(3):
        x = torch.randn(b, c.hidden, generator=g, device=device).to(torch.bfloat16)
        pos = torch.full((b, 1), t + step, dtype=torch.int64, device=device)
        st_a.seq_lens.fill_(t + step + 1)
        fused = model._attention_decode(L, 0, st_a, x, pos)
        ref = model._attention(L, 0, st_b, x[:, None], pos, True)[:, 0]
        torch.testing.assert_close(st_a.key_caches[0], st_b.key_caches[0], rtol=0, atol=0)
        torch.testing.assert_close(st_a.value_caches[0], st_b.value_caches[0], rtol=0, atol=0)
        torch.testing.assert_close(fused.float(), ref.float(), rtol=2e-2, atol=2e-2)
