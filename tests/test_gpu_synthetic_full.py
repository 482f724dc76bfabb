"""BASELINE configs[4] at full size on the GPU: the random-init
Qwen3.5-9B-shaped hybrid (32 layers, hidden 4096, full attention on HiF8 KV
every fourth layer, gated-delta-rule layers elsewhere, intermediate 12288,
vocab 151936, every projection W8A8 HiF8 static through the scheme), seeded
and calibrated on one prefill.

* layer by layer (teacher-forced: identical inputs), each of the 32 layers'
  decode path (GEMV projections, fused glue, paged decode attention or the
  fused delta-rule step) matches its prefill path (GEMM projections, torch
  glue, multi-token paged attention or the chunked delta rule);
* the logits stay finite through prefill, chunked prefill and decode, and
  decode stays as close to a whole prefill as a second, chunked prefill of
  the same tokens does (static HiF8 activation quant amplifies one-ulp
  differences over 32 random-init layers, so neither is bit-equal);
* the HIP-graph decode loop reproduces eager decoding token for token;
* under the reference's scale convention (weight rows' amax -> 1.0,
  activation and KV scales near calibrated amax / 12, so activations land in
  HiF8's 3-bit-mantissa band), decode tracks prefill tightly.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full_model(native_ops, device):
    from hif8_rocm.synthetic_model import HybridConfig, HybridModel

    print("building the full-size hybrid model (32 layers, hidden 4096)", flush=True)
    model = HybridModel(HybridConfig(), device, seed=0)
    model.calibrate(batch=1, tokens=128)
    torch.cuda.synchronize()
    yield model
    del model
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def reference_convention_model(native_ops, device):
    from hif8_rocm.synthetic_model import HybridConfig, HybridModel

    print("building the full-size hybrid model, reference scale convention", flush=True)
    model = HybridModel(HybridConfig(weight_scale_div=1.0, act_scale_div=12.0), device, seed=0)
    model.calibrate(batch=1, tokens=128)
    torch.cuda.synchronize()
    yield model
    del model
    torch.cuda.empty_cache()


def _positions(device, b, start, stop):
    return torch.arange(start, stop, device=device).expand(b, -1).contiguous()


def _cos(a, b):
    a, b = a.float().reshape(a.shape[0], -1), b.float().reshape(b.shape[0], -1)
    return float(torch.nn.functional.cosine_similarity(a, b, dim=-1).min())


def _maxrel(a, b):
    return float((a.float() - b.float()).abs().max() / b.float().abs().max())


def test_every_layer_decode_path_matches_its_prefill_path(full_model, device):
    """Teacher-forced, layer by layer, at full size: each of the 32 layers'
    mixer and MLP get the same inputs through the decode path (GEMV
    projections, fused glue, fused q/k norm + rotary + cache slots, paged
    decode attention or the fused delta-rule step) and through the prefill
    path (GEMM projections, torch glue, multi-token paged attention or the
    chunked delta rule), with the decode state built by a prefill of the
    first t - 1 rows.  The outputs are compared at the last position.  The
    attention kernels differ by up to one bf16 ulp of their output, which the
    static HiF8 quant of the o-projection input can turn into a few percent on
    single elements; everything else agrees to FP32 rounding."""
    from hif8_rocm.synthetic_model import rms_norm

    model = full_model
    c = model.cfg
    ops = torch.ops.vllm_ascend_hif8
    b, t = 2, 65
    g = torch.Generator(device=device).manual_seed(33)
    attn_i = lin_i = 0
    for i, L in enumerate(model.layers):
        x = rms_norm(torch.randn(b, t, c.hidden, generator=g, device=device).to(torch.bfloat16), L["input_norm"],
                     c.rms_eps)
        full = c.is_full_attention(i)
        st_pre, st_dec = model.new_state(b, t + 8), model.new_state(b, t + 8)
        st_pre.seq_lens.fill_(t)
        st_dec.seq_lens.fill_(t - 1)
        if full:
            pre = model._attention(L, attn_i, st_pre, x, _positions(device, b, 0, t), decode=False)[:, -1]
            model._attention(L, attn_i, st_dec, x[:, :t - 1], _positions(device, b, 0, t - 1), decode=False)
            st_dec.seq_lens.fill_(t)
            dec = model._attention_decode(L, attn_i, st_dec, x[:, -1].contiguous(),
                                          torch.full((b, 1), t - 1, device=device))
            attn_i += 1
            tol_cos, tol_rel = 0.999, 0.05
        else:
            pre = model._linear_attention(L, lin_i, st_pre, x, decode=False)[:, -1]
            model._linear_attention(L, lin_i, st_dec, x[:, :t - 1], decode=False)
            dec = model._linear_attention_decode(L, lin_i, st_dec, x[:, -1].contiguous())
            lin_i += 1
            tol_cos, tol_rel = 0.9999, 0.02
        assert bool(torch.isfinite(dec).all()) and bool(torch.isfinite(pre).all()), i
        print(f"layer {i} {'attention' if full else 'linear'}: cos {_cos(dec, pre):.6f} maxrel "
              f"{_maxrel(dec, pre):.3e}", flush=True)
        assert _cos(dec, pre) > tol_cos and _maxrel(dec, pre) < tol_rel, i
        # The MLP: torch glue over the prefill GEMMs vs the decode step's
        # fused add + RMSNorm + quant, GEMV, fused SiLU-mul + quant, GEMV.
        h = torch.randn(b, c.hidden, generator=g, device=device).to(torch.bfloat16)
        mix = torch.randn(b, c.hidden, generator=g, device=device).to(torch.bfloat16)
        resid = (h.float() + mix.float()).to(torch.bfloat16)
        pre = model._mlp(L, rms_norm(resid[:, None], L["post_norm"], c.rms_eps))[:, 0]
        _, codes, rs = ops.hif8_add_rms_norm_quant(h.clone(), mix, L["post_norm"], c.rms_eps,
                                                   L["gate_up"].layer.input_scale)
        codes, rs = ops.hif8_silu_mul_quant(L["gate_up"].from_codes(codes, rs), L["down"].layer.input_scale)
        dec = L["down"].from_codes(codes, rs)
        assert _cos(dec, pre) > 0.9999 and _maxrel(dec, pre) < 0.02, (i, _cos(dec, pre), _maxrel(dec, pre))


def _decode_vs_prefill(model, device):
    """Four decode steps after a 64-token prompt, against one prefill of the
    same 68 tokens and against a chunked prefill (64 rows, then the 4 new
    rows as one chunk).  Returns the minimum logits cosines (decode vs whole
    prefill, chunked vs whole prefill) over the batch."""
    b, t, steps = 2, 64, 4
    g = torch.Generator(device=device).manual_seed(30)
    prompt = torch.randint(0, model.cfg.vocab, (b, t), generator=g, device=device)
    st = model.new_state(b, t + steps + 1)
    st.seq_lens.fill_(t)
    logits = model.forward(st, prompt, _positions(device, b, 0, t), decode=False)
    assert bool(torch.isfinite(logits).all())
    toks = [logits.argmax(-1, keepdim=True)]
    for j in range(steps):
        st.seq_lens.add_(1)
        logits = model.forward(st, toks[-1], torch.full((b, 1), t + j, device=device), decode=True)
        assert bool(torch.isfinite(logits).all())
        toks.append(logits.argmax(-1, keepdim=True))
    full = torch.cat([prompt] + toks[:steps], dim=1)
    whole = model.new_state(b, full.shape[1])
    whole.seq_lens.fill_(full.shape[1])
    ref = model.forward(whole, full, _positions(device, b, 0, full.shape[1]), decode=False)
    chunked = model.new_state(b, full.shape[1])
    chunked.seq_lens.fill_(t)
    model.forward(chunked, prompt, _positions(device, b, 0, t), decode=False)
    chunked.seq_lens.fill_(full.shape[1])
    two = model.forward(chunked, full[:, t:], _positions(device, b, t, full.shape[1]), decode=False)
    assert bool(torch.isfinite(ref).all()) and bool(torch.isfinite(two).all())
    return _cos(logits, ref), _cos(two, ref)


def test_full_size_decode_tracks_prefill(full_model, device):
    """End to end under the default scale convention (every amax -> 32768):
    random-init weights with static HiF8 activation quant amplify one-ulp
    differences layer after layer (activations sit in HiF8's 1-mantissa-bit
    band there, a 50 % step), so after 32 layers two valid computations of
    the same logits are far from bit-equal: the yardstick is the chunked
    prefill, whose kernels are the whole prefill's own.  Decode must stay at
    least as close to the whole prefill as that chunked prefill does (minus
    0.05), and every logit must stay finite."""
    cos_dec, cos_two = _decode_vs_prefill(full_model, device)
    print(f"decode vs prefill cosine {cos_dec:.4f}; chunked vs whole prefill {cos_two:.4f}", flush=True)
    assert cos_dec > cos_two - 0.05 and cos_dec > 0.5, (cos_dec, cos_two)


def test_full_size_decode_tracks_prefill_reference_scale_convention(reference_convention_model, device):
    """The same comparison under the reference's scale convention: weight
    rows' amax -> 1.0 and activation / KV scales at calibrated amax / 12,
    which keep activations in HiF8's 3-bit-mantissa band.  Decode, chunked
    prefill and whole prefill then agree far more closely (MI355X: cosine
    0.982 and 0.980, against 0.81 and 0.80 under the default convention), and
    decode stays as close to the whole prefill as the chunked prefill does."""
    cos_dec, cos_two = _decode_vs_prefill(reference_convention_model, device)
    print(f"reference convention: decode vs prefill cosine {cos_dec:.4f}; chunked vs whole prefill "
          f"{cos_two:.4f}", flush=True)
    assert cos_dec > 0.97 and cos_dec > cos_two - 0.01, (cos_dec, cos_two)


def test_full_size_graph_replay_matches_eager(full_model, device):
    from hif8_rocm.synthetic_model import generate

    g = torch.Generator(device=device).manual_seed(32)
    prompt = torch.randint(0, full_model.cfg.vocab, (2, 64), generator=g, device=device)
    eager, _ = generate(full_model, prompt, 6, graph=False)
    graphed, timings = generate(full_model, prompt, 6, graph=True)
    assert torch.equal(eager, graphed)
    assert timings["decode_steps"] == 4
