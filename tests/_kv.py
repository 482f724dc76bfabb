"""Paged HiF8 caches for the attention tests (built on the GPU by the
bit-exact cache-write kernel, from CPU-seeded K/V)."""

from __future__ import annotations

import math

import torch

HIF8_MAX = 32768.0
# The reference's real layer-3 K / V cache scales (test_hif8_kv_npu.py:427-436).
KEY_SCALES_L3 = [0.9432383179664612, 0.7343872785568237, 0.9391698241233826, 1.1160656213760376]
VALUE_SCALES_L3 = [0.3244977593421936, 0.416015625, 0.5311850309371948, 0.3086029291152954]


def randn(shape, seed, mul=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * mul).to(dtype)


def build_cache(device, lens, hkv, d, bs, seed, dv=None, bt_dtype=torch.int32, extra_blocks=3, mixed=False,
                scales=None, kv_mul=(1.0, 1.0)):
    """Shuffled pages for each request, K/V ~ N(0, 1) * kv_mul bf16 written by the (bit-exact) write
    kernel with per-head scales absmax / 32768, or ``scales`` = (key scales, value scales) per head
    (``mixed``: every third slot with other scales)."""
    from hif8_rocm import kv_cache

    dv = d if dv is None else dv
    blocks = [math.ceil(n / bs) for n in lens]
    nb = sum(blocks) + extra_blocks
    width = max(max(blocks), 1) + 1          # a trailing -1 column beyond every request
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(nb, generator=g)
    table = torch.full((len(lens), width), -1, dtype=torch.int64)
    used = 0
    for b, nblk in enumerate(blocks):
        table[b, :nblk] = perm[used:used + nblk]
        used += nblk
    key = (torch.randn(nb * bs, hkv, d, generator=g) * kv_mul[0]).to(torch.bfloat16)
    value = (torch.randn(nb * bs, hkv, dv, generator=g) * kv_mul[1]).to(torch.bfloat16)
    if scales is None:
        ks = (key.float().abs().amax(dim=(0, 2)) / HIF8_MAX).to(device)
        vs = (value.float().abs().amax(dim=(0, 2)) / HIF8_MAX).to(device)
    else:
        ks = torch.tensor(scales[0], dtype=torch.float32, device=device)
        vs = torch.tensor(scales[1], dtype=torch.float32, device=device)
    kc = torch.zeros((nb, bs, hkv, d + 4), dtype=torch.uint8, device=device)
    vc = torch.zeros((nb, bs, hkv, dv + 4), dtype=torch.uint8, device=device)
    slots = torch.arange(nb * bs, dtype=torch.int64, device=device)
    if mixed:
        other = slots % 3 == 1
        kv_cache.write_kv_cache(key.to(device), value.to(device), kc, vc, torch.where(other, -1, slots), ks, vs)
        kv_cache.write_kv_cache(key.to(device), value.to(device), kc, vc, torch.where(other, slots, -1),
                                ks * 1.75, vs * 0.6)
    else:
        kv_cache.write_kv_cache(key.to(device), value.to(device), kc, vc, slots, ks, vs)
    return kc, vc, table.to(bt_dtype)


