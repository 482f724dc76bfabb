"""Pure-torch pieces of the synthetic hybrid model on the CPU: the chunked
gated delta rule (used for prefill) against the token-by-token recurrence
(used for decode), in float64, with a carried initial state and a length
that is not a multiple of the chunk."""

import pytest
import torch

from hif8_rocm.synthetic_model import HybridConfig, gated_delta_chunked, gated_delta_step


def _inputs(b, h, t, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(b, h, t, dk, generator=g, dtype=torch.float64), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(b, h, t, dk, generator=g, dtype=torch.float64), dim=-1)
    v = torch.randn(b, h, t, dv, generator=g, dtype=torch.float64)
    gd = -torch.rand(b, h, t, generator=g, dtype=torch.float64) * 0.5
    beta = torch.rand(b, h, t, generator=g, dtype=torch.float64)
    s0 = torch.randn(b, h, dk, dv, generator=g, dtype=torch.float64) * 0.1
    return q, k, v, gd, beta, s0


@pytest.mark.parametrize("t,chunk", [(70, 16), (64, 64), (5, 16)])
def test_chunked_gated_delta_equals_recurrence(t, chunk):
    q, k, v, gd, beta, s0 = _inputs(2, 3, t, 8, 5, seed=t)
    seq_state = s0.clone()
    seq_out = torch.stack([gated_delta_step(seq_state, q[:, :, i], k[:, :, i], v[:, :, i], gd[:, :, i],
                                            beta[:, :, i]) for i in range(t)], dim=2)
    chunk_state = s0.clone()
    out = gated_delta_chunked(q, k, v, gd, beta, chunk_state, chunk=chunk)
    torch.testing.assert_close(out, seq_out, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(chunk_state, seq_state, rtol=1e-10, atol=1e-10)


def test_recurrence_closed_form_single_token():
    # From a zero state one step stores beta * v k^T and reads beta * (q . k) v.
    q, k, v, gd, beta, _ = _inputs(1, 1, 1, 4, 3, seed=3)
    state = torch.zeros(1, 1, 4, 3, dtype=torch.float64)
    o = gated_delta_step(state, q[:, :, 0], k[:, :, 0], v[:, :, 0], gd[:, :, 0], beta[:, :, 0])
    want = beta[0, 0, 0] * (q[0, 0, 0] @ k[0, 0, 0]) * v[0, 0, 0]
    torch.testing.assert_close(o[0, 0], want)
    torch.testing.assert_close(state[0, 0], beta[0, 0, 0] * torch.outer(k[0, 0, 0], v[0, 0, 0]))


def test_config_follows_the_hybrid_layout():
    c = HybridConfig()
    full = [i for i in range(c.layers) if c.is_full_attention(i)]
    assert full == [3, 7, 11, 15, 19, 23, 27, 31]
    assert c.lin_v_width == 4096 and c.intermediate == 12288 and c.hidden == 4096
    assert (c.heads + 2 * c.kv_heads) * c.head_dim == 4096 + 2048
