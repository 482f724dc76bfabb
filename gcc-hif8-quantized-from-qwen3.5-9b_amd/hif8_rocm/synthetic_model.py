"""Synthetic decode workload: a random-init Qwen3.5-9B-shaped hybrid model
driven through the static HiF8 scheme (the reference serves the real model
through vLLM with this plugin; see scheme.py:134-211 and kv_runtime.py).

Shapes.  Hidden 4096, 32 decoder layers, full attention in every fourth layer
(``full_attention_interval`` 4, exporter.py:356; layers 3, 7, ..., 31 carry
the KV scales in the reference's calibration file), intermediate 12288.
Full attention: 16 query heads, 4 KV heads, head size 256, HiF8 KV cache
with static per-head scales.  Linear attention (gated delta rule): 16 key
heads and 32 value heads of 128 (value width 4096 = the out_proj input width
of the calibration file); causal depthwise conv of width 4 over q, k, v.  The
linear-attention head split and the rotary settings are not in the reference;
they follow the public Qwen3-Next layout.

Every projection (``qkv_proj`` = q+k+v, ``o_proj``, ``in_proj_qkvz``,
``out_proj``, ``gate_up_proj``, ``down_proj``) is a W8A8HIF8_STATIC Linear
applied through :class:`scheme.W8A8HiFloat8StaticLinearMethod`; the token
embedding is a W8A8HIF8_SOFT table (gather-decode kernel).  Norms, rotary
embedding, the conv and the recurrence, ``in_proj_ba`` and the LM head run
in PyTorch (bf16 storage, fp32 math where it accumulates), as in the
reference, where they are not part of the W8A8 set
(docs/checkpoint-format.md:23-37).

Static scales come from a calibration prefill of the same model (activation
absmax / ``act_scale_div`` per Linear input, per KV head for K and V), as the
reference's calibrator produces them offline.  The default convention maps
every amax to 32768, HiF8's largest power of two (weights too); the
reference's own maps a weight row's amax to 1.0 (codec.py:212-224) and
calibrates activation scales near amax / 12 (its calibration JSON: the
searched max_abs / scale targets are 0.5 ... 64), ``weight_scale_div=1`` and
``act_scale_div=12`` here.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import kv_cache, native, scheme

HIF8_MAX = 32768.0


@dataclass
class HybridConfig:
    hidden: int = 4096
    layers: int = 32
    full_attention_interval: int = 4
    heads: int = 16
    kv_heads: int = 4
    head_dim: int = 256
    rotary_dim: int = 64
    rope_theta: float = 10_000_000.0
    intermediate: int = 12288
    lin_k_heads: int = 16
    lin_v_heads: int = 32
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    conv_kernel: int = 4
    vocab: int = 151_936
    rms_eps: float = 1e-6
    block_size: int = 128
    weight_scale_div: float = HIF8_MAX  # weight row scale = row amax / this
    act_scale_div: float = HIF8_MAX     # Linear input / KV head scale = calibrated amax / this

    def is_full_attention(self, layer: int) -> bool:
        return layer % self.full_attention_interval == self.full_attention_interval - 1

    @property
    def lin_qk_width(self) -> int:
        return self.lin_k_heads * self.lin_k_dim

    @property
    def lin_v_width(self) -> int:
        return self.lin_v_heads * self.lin_v_dim


# --------------------------------------------------------------------------
# Gated delta rule (pure torch).  Sequential form for decode, chunked form for
# prefill; both take q, k already normalised and scaled.
# --------------------------------------------------------------------------

def gated_delta_step(state: torch.Tensor, q, k, v, g, beta) -> torch.Tensor:
    """One token of the gated delta rule, in place on ``state`` [B, H, dk, dv].

    S <- exp(g) S;  S <- S + k (beta (v - S^T k))^T;  o = S^T q.
    q, k [B, H, dk]; v [B, H, dv]; g, beta [B, H].  Returns o [B, H, dv].
    """
    state.mul_(torch.exp(g)[..., None, None])
    kv_mem = (state * k[..., :, None]).sum(dim=-2)
    delta = (v - kv_mem) * beta[..., None]
    state.add_(k[..., :, None] * delta[..., None, :])
    return (state * q[..., :, None]).sum(dim=-2)


def gated_delta_chunked(q, k, v, g, beta, state: torch.Tensor, chunk: int = 64) -> torch.Tensor:
    """The gated delta rule over T tokens in chunks (WY form); updates ``state``.

    q, k [B, H, T, dk]; v [B, H, T, dv]; g, beta [B, H, T]; state [B, H, dk, dv].
    Equal to T calls of :func:`gated_delta_step` up to rounding.
    """
    b, h, t, dk = k.shape
    dv = v.shape[-1]
    pad = (-t) % chunk
    if pad:
        q = torch.nn.functional.pad(q, (0, 0, 0, pad))
        k = torch.nn.functional.pad(k, (0, 0, 0, pad))
        v = torch.nn.functional.pad(v, (0, 0, 0, pad))
        g = torch.nn.functional.pad(g, (0, pad))
        beta = torch.nn.functional.pad(beta, (0, pad))
    n = (t + pad) // chunk
    q, k, v = (x.reshape(b, h, n, chunk, -1) for x in (q, k, v))
    g = g.reshape(b, h, n, chunk).cumsum(dim=-1)
    beta = beta.reshape(b, h, n, chunk)
    k_beta = k * beta[..., None]
    v_beta = v * beta[..., None]
    lower = torch.tril(torch.ones(chunk, chunk, dtype=torch.bool, device=k.device), diagonal=-1)
    decay = torch.exp(g[..., :, None] - g[..., None, :]).masked_fill(~torch.tril(
        torch.ones(chunk, chunk, dtype=torch.bool, device=k.device)), 0.0)
    kt = k.transpose(-1, -2).contiguous()
    # T = (I + L)^-1 with L the strictly lower part of (k_beta k^T) * decay.
    lmat = (torch.matmul(k_beta, kt) * decay).masked_fill(~lower, 0.0)
    eye = torch.eye(chunk, dtype=k.dtype, device=k.device).expand_as(lmat)
    tmat = torch.linalg.solve_triangular(eye + lmat, eye.contiguous(), upper=False, unitriangular=True)
    u = torch.matmul(tmat, v_beta)                                  # [B, H, N, C, dv]
    w = torch.matmul(tmat, k_beta * torch.exp(g)[..., None])        # [B, H, N, C, dk]
    intra = torch.matmul(q, kt) * decay                             # causal, diagonal included
    out = torch.empty(b, h, n, chunk, dv, dtype=v.dtype, device=v.device)
    for i in range(n):
        s = state
        v_new = u[:, :, i] - torch.matmul(w[:, :, i], s)
        o_inter = torch.matmul(q[:, :, i] * torch.exp(g[:, :, i])[..., None], s)
        out[:, :, i] = o_inter + torch.matmul(intra[:, :, i], v_new)
        g_last = g[:, :, i, -1]
        k_decay = k[:, :, i] * torch.exp(g_last[..., None] - g[:, :, i])[..., None]
        state.mul_(torch.exp(g_last)[..., None, None])
        state.add_(torch.matmul(k_decay.transpose(-1, -2).contiguous(), v_new))
    return out.reshape(b, h, n * chunk, dv)[:, :, :t]


# --------------------------------------------------------------------------
# Building blocks
# --------------------------------------------------------------------------

def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (y * weight.float()).to(x.dtype)


class StaticLinear:
    """A W8A8HIF8_STATIC Linear of random N(0, 0.02) weights, per-channel
    HiF8 codes made by the static quant kernel (absmax -> 2^15 per row).
    During calibration each call sets the input scale from the running
    activation absmax before applying the scheme."""

    def __init__(self, n: int, k: int, device, generator: torch.Generator, std: float = 0.02,
                 weight_div: float = HIF8_MAX, act_div: float = HIF8_MAX):
        codes = torch.empty(n, k, dtype=torch.uint8, device=device)
        scales = torch.empty(n, dtype=torch.float32, device=device)
        step = max(1, (64 << 20) // (k * 2))
        for r in range(0, n, step):
            w = (torch.randn(min(step, n - r), k, generator=generator, device=device) * std).to(torch.bfloat16)
            s = (w.float().abs().amax(dim=1) / weight_div).clamp_min(1e-30)
            c, _ = native.static_quant(w, s)
            codes[r:r + w.shape[0]] = c
            scales[r:r + w.shape[0]] = s
        self.layer = torch.nn.Module()
        self.layer.weight = torch.nn.Parameter(codes, requires_grad=False)
        self.layer.weight_scale = torch.nn.Parameter(scales.reshape(n, 1), requires_grad=False)
        self.layer.input_scale = torch.nn.Parameter(torch.ones(1, dtype=torch.float32, device=device),
                                                    requires_grad=False)
        self.method = scheme.W8A8HiFloat8StaticLinearMethod()
        self.method.process_weights_after_loading(self.layer)
        self.amax = torch.zeros((), dtype=torch.float32, device=device)
        self.act_div = act_div
        self.calibrating = False

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if self.calibrating:
            self.amax = torch.maximum(self.amax, x.float().abs().amax())
            self.layer.input_scale.data.copy_((self.amax / self.act_div).clamp_min(1e-30).reshape(1))
        return self.method.apply(self.layer, x)

    def from_codes(self, codes: torch.Tensor, row_scale: torch.Tensor) -> torch.Tensor:
        """The projection of activations a producer kernel already quantized
        with this layer's input scale: the GEMV / GEMM half of ``__call__``,
        routed as the scheme routes it."""
        decoded = getattr(self.layer, "_hif8_weight_bf16", None)
        if decoded is not None and codes.numel() // codes.shape[-1] > 4:
            return native.soft_linear_decoded_weight(codes, decoded, row_scale, self.layer.weight_scale, None,
                                                     output_dtype=torch.bfloat16)
        return native.soft_linear(codes, self.layer.weight, row_scale, self.layer.weight_scale, None,
                                  output_dtype=torch.bfloat16)

    def silu_mul_quant_from_codes(self, codes: torch.Tensor, row_scale: torch.Tensor,
                                  next_input_scale: torch.Tensor):
        """For a gate_up projection (gate rows, then up rows): the static
        HiF8 codes and row scales of silu(gate) * up for the next projection,
        from activation codes of at most four rows, in one GEMV launch where
        the kernel plan allows it (the same codes as ``from_codes`` followed
        by ``hif8_silu_mul_quant``)."""
        return torch.ops.vllm_ascend_hif8.hif8_gate_up_silu_mul_quant(
            codes, self.layer.weight, row_scale.reshape(-1), self.layer.weight_scale.reshape(-1), next_input_scale)

    def conv_from_codes(self, codes: torch.Tensor, row_scale: torch.Tensor, conv_weight: torch.Tensor,
                        conv_state: torch.Tensor):
        """For a qkvz projection of at most four rows: (the bf16 projection,
        the float32 causal-conv outputs of its first conv_weight.shape[0]
        columns), the conv state shifted in place; the conv runs in the GEMV
        epilogue where the kernel plan allows it (the conv of
        ``hif8_gdn_decode_step``)."""
        return torch.ops.vllm_ascend_hif8.hif8_linear_conv(
            codes, self.layer.weight, row_scale.reshape(-1), self.layer.weight_scale.reshape(-1), conv_weight,
            conv_state)


@dataclass
class RequestState:
    """Per-batch decode state: KV caches of the attention layers, conv and
    recurrent state of the linear-attention layers, positions."""

    key_caches: list = field(default_factory=list)
    value_caches: list = field(default_factory=list)
    conv_states: list = field(default_factory=list)
    rec_states: list = field(default_factory=list)
    block_table: torch.Tensor | None = None
    seq_lens: torch.Tensor | None = None
    max_len: int = 0


class HybridModel:
    def __init__(self, cfg: HybridConfig, device, seed: int = 0):
        self.cfg = cfg
        self.calibrating = False
        # Decode quantizes projection inputs inside the glue kernels; False
        # runs the scheme's own quant per projection (same codes, more launches).
        self.fuse_input_quant = True
        # Decode runs the linear-attention mixer as the conv-epilogue qkvz GEMV
        # + one block per value head where the shapes allow; False keeps the
        # per-group kernel that folds the conv in.
        self.head_split = True
        self.device = torch.device(device)
        g = torch.Generator(device=self.device).manual_seed(seed)
        c = cfg
        div = {"weight_div": c.weight_scale_div, "act_div": c.act_scale_div}
        # SOFT embedding: HiF8 rows + per-row scales.
        emb = StaticLinear(c.vocab, c.hidden, device, g, **div)
        self.embed = torch.nn.Module()
        self.embed.weight = emb.layer.weight
        self.embed.weight_scale = emb.layer.weight_scale
        self.embed_method = scheme.W8A8HiFloat8SoftLinearMethod()
        self.embed_method.process_weights_after_loading(self.embed)
        del emb
        self.layers = []
        for i in range(c.layers):
            L = {"input_norm": torch.ones(c.hidden, dtype=torch.bfloat16, device=device),
                 "post_norm": torch.ones(c.hidden, dtype=torch.bfloat16, device=device),
                 "gate_up": StaticLinear(2 * c.intermediate, c.hidden, device, g, **div),
                 "down": StaticLinear(c.hidden, c.intermediate, device, g, **div)}
            if c.is_full_attention(i):
                L["qkv"] = StaticLinear((c.heads + 2 * c.kv_heads) * c.head_dim, c.hidden, device, g, **div)
                L["o"] = StaticLinear(c.hidden, c.heads * c.head_dim, device, g, **div)
                L["q_norm"] = torch.ones(c.head_dim, dtype=torch.bfloat16, device=device)
                L["k_norm"] = torch.ones(c.head_dim, dtype=torch.bfloat16, device=device)
                L["k_scale"] = torch.ones(c.kv_heads, dtype=torch.float32, device=device)
                L["v_scale"] = torch.ones(c.kv_heads, dtype=torch.float32, device=device)
                L["k_amax"] = torch.zeros(c.kv_heads, dtype=torch.float32, device=device)
                L["v_amax"] = torch.zeros(c.kv_heads, dtype=torch.float32, device=device)
            else:
                L["qkvz"] = StaticLinear(2 * c.lin_qk_width + 2 * c.lin_v_width, c.hidden, device, g, **div)
                L["ba"] = (torch.randn(2 * c.lin_v_heads, c.hidden, generator=g, device=device) * 0.02).to(
                    torch.bfloat16)
                L["conv"] = (torch.randn(2 * c.lin_qk_width + c.lin_v_width, c.conv_kernel, generator=g,
                                         device=device) * 0.3).to(torch.bfloat16)
                L["A_log"] = torch.log(torch.empty(c.lin_v_heads, device=device).uniform_(1, 16, generator=g))
                L["dt_bias"] = torch.ones(c.lin_v_heads, device=device)
                L["out_norm"] = torch.ones(c.lin_v_dim, dtype=torch.bfloat16, device=device)
                L["out"] = StaticLinear(c.hidden, c.lin_v_width, device, g, **div)
            self.layers.append(L)
        self.final_norm = torch.ones(c.hidden, dtype=torch.bfloat16, device=device)
        self.lm_head = (torch.randn(c.vocab, c.hidden, generator=g, device=device) * 0.02).to(torch.bfloat16)
        inv = 1.0 / (c.rope_theta ** (torch.arange(0, c.rotary_dim, 2, device=device).float() / c.rotary_dim))
        self.inv_freq = inv
        self.calibrating = False

    # ---------------------------------------------------------------- state
    def new_state(self, batch: int, max_len: int) -> RequestState:
        c = self.cfg
        blocks_per_req = (max_len + c.block_size - 1) // c.block_size
        st = RequestState(max_len=max_len)
        st.block_table = torch.arange(batch * blocks_per_req, dtype=torch.int32,
                                      device=self.device).reshape(batch, blocks_per_req)
        st.seq_lens = torch.zeros(batch, dtype=torch.int32, device=self.device)
        for i, L in enumerate(self.layers):
            if c.is_full_attention(i):
                layout = kv_cache.Hif8KVCacheLayout(num_blocks=batch * blocks_per_req, block_size=c.block_size,
                                                    num_kv_heads=c.kv_heads, head_size=c.head_dim)
                kc, vc = layout.allocate(self.device)
                st.key_caches.append(kc)
                st.value_caches.append(vc)
            else:
                st.conv_states.append(torch.zeros(batch, 2 * c.lin_qk_width + c.lin_v_width, c.conv_kernel - 1,
                                                  dtype=torch.bfloat16, device=self.device))
                st.rec_states.append(torch.zeros(batch, c.lin_v_heads, c.lin_k_dim, c.lin_v_dim,
                                                 dtype=torch.float32, device=self.device))
        return st

    def set_calibrating(self, on: bool) -> None:
        self.calibrating = on
        for L in self.layers:
            for v in L.values():
                if isinstance(v, StaticLinear):
                    v.calibrating = on

    # --------------------------------------------------------------- pieces
    def _rope(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """Rotary embedding on the first rotary_dim dims (neox halves); x [..., T, H, D], pos [..., T]."""
        rd = self.cfg.rotary_dim
        ang = pos.float()[..., None] * self.inv_freq                   # [..., T, rd/2]
        cos = torch.cos(ang)[..., None, :]
        sin = torch.sin(ang)[..., None, :]
        xr = x[..., :rd].float()
        x1, x2 = xr[..., : rd // 2], xr[..., rd // 2:]
        rot = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)
        return torch.cat([rot.to(x.dtype), x[..., rd:]], dim=-1)

    def _slots(self, st: RequestState, pos: torch.Tensor) -> torch.Tensor:
        """Flat cache slots of positions pos [B, T] (block_table row b)."""
        bs = self.cfg.block_size
        blk = torch.gather(st.block_table.long(), 1, (pos // bs).long())
        return (blk * bs + pos % bs).reshape(-1)

    def _attention_decode(self, L, idx: int, st: RequestState, x: torch.Tensor, pos: torch.Tensor, xq=None):
        """One decode token of full attention: fused q/k norm + rotary + slots,
        fused KV write, paged HiF8 decode attention; x [B, H], pos [B, 1];
        xq: x already quantized for the qkv projection (codes, row scales)."""
        c = self.cfg
        b = x.shape[0]
        qkv = L["qkv"](x) if xq is None else L["qkv"].from_codes(*xq)
        q, k, v, slots = torch.ops.vllm_ascend_hif8.hif8_qk_norm_rope(
            qkv, L["q_norm"], L["k_norm"], pos.reshape(b), self.inv_freq, st.block_table, c.block_size, c.heads,
            c.kv_heads, c.head_dim, c.rms_eps)
        kc, vc = st.key_caches[idx], st.value_caches[idx]
        kv_cache.write_kv_cache(k, v, kc, vc, slots, L["k_scale"], L["v_scale"], validate=False)
        o = kv_cache.paged_decode_attention(q, kc, vc, st.block_table, st.seq_lens, scale=1.0 / math.sqrt(c.head_dim),
                                            max_seq_len=st.max_len, validate=False)
        return L["o"](o.reshape(b, c.heads * c.head_dim))

    def _attention(self, L, idx: int, st: RequestState, h: torch.Tensor, pos: torch.Tensor, decode: bool):
        c = self.cfg
        b, t, _ = h.shape
        qkv = L["qkv"](h.reshape(b * t, -1)).reshape(b, t, -1)
        q, k, v = qkv.split([c.heads * c.head_dim, c.kv_heads * c.head_dim, c.kv_heads * c.head_dim], dim=-1)
        q = rms_norm(q.reshape(b, t, c.heads, c.head_dim), L["q_norm"], c.rms_eps)
        k = rms_norm(k.reshape(b, t, c.kv_heads, c.head_dim), L["k_norm"], c.rms_eps)
        v = v.reshape(b, t, c.kv_heads, c.head_dim)
        q = self._rope(q, pos)
        k = self._rope(k, pos)
        if self.calibrating:
            L["k_amax"] = torch.maximum(L["k_amax"], k.float().abs().amax(dim=(0, 1, 3)))
            L["v_amax"] = torch.maximum(L["v_amax"], v.float().abs().amax(dim=(0, 1, 3)))
            L["k_scale"] = (L["k_amax"] / c.act_scale_div).clamp_min(1e-30)
            L["v_scale"] = (L["v_amax"] / c.act_scale_div).clamp_min(1e-30)
        kc, vc = st.key_caches[idx], st.value_caches[idx]
        kv_cache.write_kv_cache(k.reshape(b * t, c.kv_heads, c.head_dim).contiguous(),
                                v.reshape(b * t, c.kv_heads, c.head_dim).contiguous(), kc, vc,
                                self._slots(st, pos), L["k_scale"], L["v_scale"], validate=not decode)
        scale = 1.0 / math.sqrt(c.head_dim)
        if decode:
            o = kv_cache.paged_decode_attention(q.reshape(b, c.heads, c.head_dim).contiguous(), kc, vc,
                                                st.block_table, st.seq_lens, scale=scale, max_seq_len=st.max_len,
                                                validate=False)
            o = o.reshape(b, 1, c.heads * c.head_dim)
        else:
            # Prefill or a continued (chunked) prefill: the t new rows of each
            # request are its last t positions of st.seq_lens cached tokens,
            # attended with the right-aligned causal mask over the HiF8 pages
            # (pages decoded inside the kernel, as for decode).
            o = kv_cache.paged_attention(q.reshape(b * t, c.heads, c.head_dim).contiguous(), kc, vc,
                                         st.block_table, st.seq_lens, scale=scale, query_lens=[t] * b,
                                         max_query_len=t, max_seq_len=st.max_len, validate=False)
            o = o.reshape(b, t, c.heads * c.head_dim)
        return L["o"](o.reshape(b * t, -1)).reshape(b, t, -1)

    def _linear_attention(self, L, idx: int, st: RequestState, h: torch.Tensor, decode: bool):
        c = self.cfg
        b, t, _ = h.shape
        qkvz = L["qkvz"](h.reshape(b * t, -1)).reshape(b, t, -1)
        mixed, z = qkvz.split([2 * c.lin_qk_width + c.lin_v_width, c.lin_v_width], dim=-1)
        ba = torch.nn.functional.linear(h.reshape(b * t, -1), L["ba"]).float().reshape(b, t, -1)
        beta = torch.sigmoid(ba[..., : c.lin_v_heads])
        gdecay = -torch.exp(L["A_log"]) * torch.nn.functional.softplus(ba[..., c.lin_v_heads:] + L["dt_bias"])
        # Causal depthwise conv over time with the carried state (width conv_kernel).
        conv_state = st.conv_states[idx]
        seq = torch.cat([conv_state, mixed.transpose(1, 2)], dim=-1)           # [B, C, K-1+T]
        w = L["conv"].float()
        acc = sum(seq[..., j: j + t].float() * w[:, j: j + 1] for j in range(c.conv_kernel))
        conv_state.copy_(seq[..., -(c.conv_kernel - 1):])
        mixed = torch.nn.functional.silu(acc).transpose(1, 2)                  # [B, T, C]
        q, k, v = mixed.split([c.lin_qk_width, c.lin_qk_width, c.lin_v_width], dim=-1)
        rep = c.lin_v_heads // c.lin_k_heads
        q = q.reshape(b, t, c.lin_k_heads, c.lin_k_dim).repeat_interleave(rep, dim=2)
        k = k.reshape(b, t, c.lin_k_heads, c.lin_k_dim).repeat_interleave(rep, dim=2)
        v = v.reshape(b, t, c.lin_v_heads, c.lin_v_dim)
        q = torch.nn.functional.normalize(q, dim=-1) / math.sqrt(c.lin_k_dim)
        k = torch.nn.functional.normalize(k, dim=-1)
        state = st.rec_states[idx]
        if decode:
            o = gated_delta_step(state, q[:, 0], k[:, 0], v[:, 0], gdecay[:, 0], beta[:, 0])[:, None]
        else:
            o = gated_delta_chunked(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                    gdecay.transpose(1, 2), beta.transpose(1, 2), state).transpose(1, 2)
        zz = z.reshape(b, t, c.lin_v_heads, c.lin_v_dim)
        o = rms_norm(o, L["out_norm"], c.rms_eps).float() * torch.nn.functional.silu(zz.float())
        o = o.to(h.dtype).reshape(b * t, c.lin_v_width)
        return L["out"](o).reshape(b, t, -1)

    def _linear_attention_decode(self, L, idx: int, st: RequestState, x: torch.Tensor, xq=None) -> torch.Tensor:
        """One decode token of the linear-attention mixer with the fused glue
        kernel (b/a projection + conv + recurrence + gated norm in one launch
        where the head shapes allow it); x [B, H]; xq: x already quantized
        for the qkvz projection."""
        c = self.cfg
        ops = torch.ops.vllm_ascend_hif8
        if xq is not None and self._head_split_ok(x.shape[0]):
            # Two launches: the qkvz GEMV with the conv in its epilogue, then
            # one block per (request, value head) for the recurrence.
            qkvz, conv = L["qkvz"].conv_from_codes(*xq, L["conv"], st.conv_states[idx])
            o = ops.hif8_gdn_decode_head(conv, qkvz, x, L["ba"], L["A_log"], L["dt_bias"], st.rec_states[idx],
                                         L["out_norm"], c.lin_k_heads, c.lin_v_heads, c.lin_k_dim, c.lin_v_dim,
                                         c.rms_eps)
            return L["out"](o)
        qkvz = L["qkvz"](x) if xq is None else L["qkvz"].from_codes(*xq)
        o = ops.hif8_gdn_decode_token(
            qkvz, x, L["ba"], L["conv"], st.conv_states[idx], L["A_log"], L["dt_bias"], st.rec_states[idx],
            L["out_norm"], c.lin_k_heads, c.lin_v_heads, c.lin_k_dim, c.lin_v_dim, c.rms_eps)
        return L["out"](o)

    def _head_split_ok(self, batch: int) -> bool:
        """Whether the decode token's linear-attention mixer takes the
        conv-epilogue GEMV + per-head kernel pair (the shapes that pair
        handles; others run the fused per-group kernel)."""
        c = self.cfg
        return (self.head_split and batch <= 4 and 2 <= c.conv_kernel <= 4 and c.lin_k_dim in (32, 64, 128)
                and c.lin_v_dim <= 128 and c.hidden % 8 == 0 and c.hidden <= 8192)

    def _fuse_input_quant(self) -> bool:
        """Whether the decode step quantizes projection inputs inside the
        norm and SiLU-mul kernels (same codes as the scheme's own quant)."""
        c = self.cfg
        return (self.fuse_input_quant and not self.calibrating and scheme._static_scale_factor() == 1.0
                and c.hidden % 8 == 0 and c.hidden <= 8192 and c.intermediate % 8 == 0)

    def _forward_decode(self, st: RequestState, ids: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """The decode step with fused glue: residual add + RMSNorm in one
        kernel, SiLU-mul in one, the linear-attention token in two; the input
        quant of the qkv / qkvz, gate_up and down projections runs inside the
        norm and SiLU-mul kernels (``fuse_input_quant``)."""
        c = self.cfg
        ops = torch.ops.vllm_ascend_hif8
        b = ids.shape[0]
        h = native.embedding_lookup(self.embed.weight, self.embed.weight_scale, ids.reshape(b),
                                    validate=False).reshape(b, c.hidden)
        pending = None
        attn_i = lin_i = 0
        fuse = self._fuse_input_quant()
        for i, L in enumerate(self.layers):
            full = c.is_full_attention(i)
            xq = None
            if fuse:
                proj = L["qkv"] if full else L["qkvz"]
                x, codes, rs = ops.hif8_add_rms_norm_quant(h, pending, L["input_norm"], c.rms_eps,
                                                           proj.layer.input_scale)
                xq = (codes, rs)
            else:
                x = ops.hif8_add_rms_norm(h, pending, L["input_norm"], c.rms_eps)
            if full:
                mix = self._attention_decode(L, attn_i, st, x, pos, xq)
                attn_i += 1
            else:
                mix = self._linear_attention_decode(L, lin_i, st, x, xq)
                lin_i += 1
            if fuse:
                _, codes, rs = ops.hif8_add_rms_norm_quant(h, mix, L["post_norm"], c.rms_eps,
                                                           L["gate_up"].layer.input_scale)
                codes, rs = L["gate_up"].silu_mul_quant_from_codes(codes, rs, L["down"].layer.input_scale)
                pending = L["down"].from_codes(codes, rs)
            else:
                x2 = ops.hif8_add_rms_norm(h, mix, L["post_norm"], c.rms_eps)
                pending = L["down"](ops.hif8_silu_mul(L["gate_up"](x2)))
        last = ops.hif8_add_rms_norm(h, pending, self.final_norm, c.rms_eps)
        return self._lm_head(last)

    def _lm_head(self, last: torch.Tensor) -> torch.Tensor:
        """bf16 logits of the last positions [B, H] -> float32 [B, vocab]: up to
        four rows through the library's bf16 GEMV (the 1.24 GB head streamed
        at 6.2 TB/s, 202 us at B = 1 against 250 us for torch's GEMM on
        MI355X), more through torch."""
        if last.shape[0] <= 4:
            return torch.ops.vllm_ascend_hif8.hif8_bf16_gemv(last.contiguous(), self.lm_head).float()
        return torch.nn.functional.linear(last, self.lm_head).float()

    def _mlp(self, L, h: torch.Tensor) -> torch.Tensor:
        c = self.cfg
        b, t, _ = h.shape
        gu = L["gate_up"](h.reshape(b * t, -1))
        gate, up = gu.split([c.intermediate, c.intermediate], dim=-1)
        act = (torch.nn.functional.silu(gate.float()) * up.float()).to(h.dtype)
        return L["down"](act).reshape(b, t, -1)

    # -------------------------------------------------------------- forward
    def forward(self, st: RequestState, ids: torch.Tensor, pos: torch.Tensor, decode: bool) -> torch.Tensor:
        """ids, pos [B, T] (T = 1 when decode); returns the last position's logits [B, vocab] (fp32).

        The caller sets ``st.seq_lens`` to the lengths including these tokens
        before the call: the attention layers read them, and the T rows of a
        prefill are the last T positions of those lengths (so a prefill may
        continue a request whose earlier tokens are already cached)."""
        c = self.cfg
        if decode:
            return self._forward_decode(st, ids, pos)
        # A prefill is never graph-captured, so the lengths can be checked
        # here: the T rows are the last T positions of st.seq_lens, so each
        # length must be the last position + 1 (a stale st.seq_lens would give
        # rows that see no keys, i.e. silent zero attention).
        want = pos[:, -1].to(torch.int64) + 1
        if st.seq_lens is None or not torch.equal(st.seq_lens[:pos.shape[0]].to(torch.int64), want):
            raise ValueError("st.seq_lens must hold each request's length including these tokens "
                             "(the last position + 1) before a prefill forward")
        h = self.embed_method.embedding(self.embed, ids)
        attn_i = lin_i = 0
        for i, L in enumerate(self.layers):
            x = rms_norm(h, L["input_norm"], c.rms_eps)
            if c.is_full_attention(i):
                h = h + self._attention(L, attn_i, st, x, pos, decode)
                attn_i += 1
            else:
                h = h + self._linear_attention(L, lin_i, st, x, decode)
                lin_i += 1
            h = h + self._mlp(L, rms_norm(h, L["post_norm"], c.rms_eps))
        last = rms_norm(h[:, -1], self.final_norm, c.rms_eps)
        return self._lm_head(last)

    def calibrate(self, batch: int = 1, tokens: int = 64, seed: int = 1) -> None:
        """Static scales from one prefill of random tokens: each Linear's input
        scale follows the running activation absmax, K/V scales the per-head absmax."""
        g = torch.Generator(device=self.device).manual_seed(seed)
        st = self.new_state(batch, tokens)
        ids = torch.randint(0, self.cfg.vocab, (batch, tokens), generator=g, device=self.device)
        pos = torch.arange(tokens, device=self.device).expand(batch, tokens).contiguous()
        st.seq_lens.fill_(tokens)
        self.set_calibrating(True)
        try:
            self.forward(st, ids, pos, decode=False)
        finally:
            self.set_calibrating(False)
        del st


def generate(model: HybridModel, prompt: torch.Tensor, new_tokens: int, graph: bool = True):
    """Greedy decode of ``new_tokens`` after the prompt [B, T].

    Returns (tokens [B, new_tokens], timings) with timings in seconds:
    ``prefill`` (prompt forward + first token), ``setup`` (the first decode
    step, run eagerly, and the graph recording), ``decode`` (the remaining
    ``decode_steps`` steps).  With ``graph`` the decode step is recorded once
    as a HIP graph and replayed; positions, lengths and the input token live
    in device tensors updated in place."""
    b, t = prompt.shape
    dev = model.device
    st = model.new_state(b, t + new_tokens)
    pos = torch.arange(t, device=dev).expand(b, t).contiguous()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record()
    st.seq_lens.fill_(t)
    logits = model.forward(st, prompt, pos, decode=False)
    tok = logits.argmax(dim=-1, keepdim=True).to(torch.int64)
    ev[1].record()
    out = torch.empty(b, new_tokens, dtype=torch.int64, device=dev)
    out[:, 0:1] = tok
    cur = tok.clone()
    cur_pos = torch.full((b, 1), t, dtype=torch.int64, device=dev)

    def step():
        st.seq_lens.add_(1)
        lg = model.forward(st, cur, cur_pos, decode=True)
        cur.copy_(lg.argmax(dim=-1, keepdim=True))
        cur_pos.add_(1)

    first = 1
    replay = None
    if new_tokens > 1:
        # The first decode step runs eagerly (it also warms the allocator);
        # the graph is recorded after it (recording executes nothing).
        step()
        out[:, 1:2] = cur
        first = 2
        if graph:
            replay = torch.cuda.CUDAGraph()
            with torch.cuda.graph(replay):
                step()
    ev[2].record()
    for i in range(first, new_tokens):
        if replay is not None:
            replay.replay()
        else:
            step()
        out[:, i:i + 1] = cur
    ev[3].record()
    ev[3].synchronize()
    timings = {"prefill": ev[0].elapsed_time(ev[1]) / 1e3, "setup": ev[1].elapsed_time(ev[2]) / 1e3,
               "decode": ev[2].elapsed_time(ev[3]) / 1e3, "decode_steps": max(0, new_tokens - first)}
    return out, timings
