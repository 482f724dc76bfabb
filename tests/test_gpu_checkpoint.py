"""A synthetic exported checkpoint loaded onto the GPU and run through the
static Linear (fused q/k/v, gate/up) and the SOFT embedding, against the
oracle on the same tensors (rtol = atol = 1e-2 for the Linear, bit-exact for
the embedding)."""

import numpy as np
import pytest
import torch

from _checkpoint import ATTN, EMBED, GATE_UP, HIDDEN, MLP, QKV, VOCAB, write_checkpoint
from _data import bf16_activation
from oracle import hif8_oracle as o

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows", [1, 4, 64])
@pytest.mark.parametrize("group", ["qkv", "gate_up"])
def test_checkpoint_static_linear_matches_oracle(native_ops, device, tmp_path, rows, group):
    from hif8_rocm.checkpoint import Hif8Checkpoint

    tensors = write_checkpoint(tmp_path)
    prefix, comps = (ATTN, QKV) if group == "qkv" else (MLP, GATE_UP)
    names = [f"{prefix}.{n}" for n in comps]
    layer = Hif8Checkpoint.open(tmp_path).static_linear(names, device)
    x = bf16_activation(rows, HIDDEN, seed=rows * 31 + len(group))
    y = layer.quant_method.apply(layer, x.to(device))
    scale = tensors[f"{names[0]}.input_scale"].numpy()
    xq, _ = o.static_quant_rows(x.float().numpy(), scale)
    want = np.concatenate([
        o.linear_u8_u8(xq, np.repeat(scale, rows), tensors[f"{n}.weight"].numpy(),
                       tensors[f"{n}.weight_scale"].numpy().reshape(-1))
        for n in names], axis=1)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (rows, sum(comps.values()))
    torch.testing.assert_close(y.cpu().float(), torch.from_numpy(want.astype(np.float32)), rtol=1e-2, atol=1e-2)


def test_checkpoint_embedding_matches_oracle(native_ops, device, tmp_path):
    from hif8_rocm.checkpoint import Hif8Checkpoint

    tensors = write_checkpoint(tmp_path)
    emb = Hif8Checkpoint.open(tmp_path).embedding(EMBED, device)
    ids = torch.tensor([[0, 5, VOCAB - 1], [17, 17, 2]], dtype=torch.int64)
    out = emb.quant_method.embedding(emb, ids.to(device))
    want = o.embedding_reference(tensors[f"{EMBED}.weight"].numpy(),
                                 tensors[f"{EMBED}.weight_scale"].numpy().reshape(-1), ids.numpy())
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (2, 3, HIDDEN)
    torch.testing.assert_close(out.cpu().float().reshape(-1, HIDDEN), torch.from_numpy(want),
                               rtol=0, atol=0, equal_nan=True)
