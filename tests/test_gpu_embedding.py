"""HiF8 token-embedding gather-decode on the GPU against the oracle
(scheme.py:121-131 semantics): bit-exact bf16, NaN where the oracle has NaN."""

import numpy as np
import pytest
import torch

from oracle import hif8_oracle as o

pytestmark = pytest.mark.gpu


def _check(got: torch.Tensor, want: np.ndarray):
    g = got.cpu().float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(g), nan)
    assert np.array_equal(g[~nan].view(np.uint32), want[~nan].astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("dim", [4096, 100, 16])
@pytest.mark.parametrize("id_dtype", [torch.int32, torch.int64])
def test_embedding_matches_oracle(native_ops, device, dim, id_dtype):
    from hif8_rocm import native

    rng = np.random.default_rng(dim)
    vocab = 1000
    weight = rng.integers(0, 256, (vocab, dim), dtype=np.uint8)   # every code incl. NaN / Inf
    scale = (rng.random(vocab, dtype=np.float32) * 2.0 + 1e-4).astype(np.float32)
    scale[:3] = [1.0, 7.3e-6, 3.0e4]
    ids = rng.integers(0, vocab, (4, 9))
    ids[0, :3] = [0, 1, 2]
    out = native.embedding_lookup(torch.from_numpy(weight).to(device), torch.from_numpy(scale).to(device),
                                  torch.from_numpy(ids).to(id_dtype).to(device))
    torch.cuda.synchronize()
    assert out.shape == (4, 9, dim) and out.dtype == torch.bfloat16
    _check(out.reshape(-1, dim), o.embedding_reference(weight, scale, ids))


def test_embedding_method_and_invalid_ids(native_ops, device):
    from hif8_rocm import native, scheme

    rng = np.random.default_rng(3)
    layer = torch.nn.Module()
    layer.weight = torch.nn.Parameter(torch.from_numpy(rng.integers(0, 111, (64, 256), dtype=np.uint8)).to(device),
                                      requires_grad=False)
    layer.weight_scale = torch.nn.Parameter(torch.rand(64, 1, device=device) + 0.5, requires_grad=False)
    method = scheme.W8A8HiFloat8SoftEmbeddingMethod()
    method.process_weights_after_loading(layer)
    ids = torch.tensor([[5, 63, 0]], device=device)
    out = method.embedding(layer, ids)
    _check(out.reshape(-1, 256), o.embedding_reference(layer.weight.cpu().numpy(), layer.weight_scale.cpu().numpy(),
                                                       ids.cpu().numpy()))
    with pytest.raises(IndexError):
        method.embedding(layer, torch.tensor([1, 64], device=device))
    quiet = native.embedding_lookup(layer.weight, layer.weight_scale, torch.tensor([64, -1, 2], device=device),
                                    validate=False)
    torch.cuda.synchronize()
    assert not quiet[:2].float().any()
    _check(quiet[2:], o.embedding_reference(layer.weight.cpu().numpy(), layer.weight_scale.cpu().numpy(),
                                            np.array([2])))
