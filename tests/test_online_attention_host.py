"""Argument checks of the op-level API (online_attention.py:42-63, 89-147) that need no
GPU: the reference's ValueErrors come first, and valid host tensors are refused with
UnsupportedAttentionBackend rather than computed on the CPU."""

import pytest
import torch

import aster_amd
from aster_amd import AttentionBlock, QuantizedKV, SoftmaxState, UnsupportedAttentionBackend


def _block(offset=0, length=16, batch=1, heads=2, dim=64, dtype=torch.float32, padding=None):
    codes = torch.zeros(batch, heads, length, dim, dtype=torch.int8)
    scales = torch.ones(batch, heads, length, 1)
    kv = QuantizedKV(codes, scales, dtype)
    return AttentionBlock(kv, kv, offset, padding)


def _call(query=None, blocks=None, positions=None, **kw):
    query = torch.zeros(1, 4, 2, 64) if query is None else query
    blocks = [_block()] if blocks is None else blocks
    positions = torch.tensor([[0, 5]]) if positions is None else positions
    return aster_amd.online_attention(query, blocks, query_positions=positions, **kw)


@pytest.mark.parametrize("kwargs,message", [
    (dict(blocks=[]), "Need nonempty"),
    (dict(query=torch.zeros(1, 4, 2)), "Need nonempty"),
    (dict(query_block_size=0), "Need nonempty"),
    (dict(query=torch.full((1, 4, 2, 64), float("nan"))), "Query must be finite"),
    (dict(causal=1), "Invalid causal/window"),
    (dict(window=0), "Invalid causal/window"),
    (dict(positions=torch.tensor([[0, -1]])), "Query positions"),
    (dict(positions=torch.tensor([[0.0, 1.0]])), "Query positions"),
    (dict(query_padding=torch.tensor([[0, 2]])), "query padding"),
    (dict(query=torch.zeros(1, 3, 2, 64)), "divide into KV groups"),
    (dict(blocks=[_block(dim=32)]), "layout/dtype/device"),
    (dict(blocks=[_block(dtype=torch.float16)]), "layout/dtype/device"),
    (dict(blocks=[_block(padding=torch.ones(1, 15))]), "key padding"),
    (dict(blocks=[_block(0, 16), _block(10, 16)]), "Overlapping"),
    (dict(scale=float("inf")), "scale must be finite"),
])
def test_reference_value_errors(kwargs, message):
    with pytest.raises(ValueError, match=message):
        _call(**kwargs)


def test_non_finite_pages_are_rejected():
    block = _block()
    bad = QuantizedKV(block.key.values, torch.zeros_like(block.key.scales), torch.float32)
    with pytest.raises(ValueError, match="finite values"):
        _call(blocks=[AttentionBlock(bad, block.value, 0)])


def test_valid_host_tensors_are_refused_not_computed():
    with pytest.raises(UnsupportedAttentionBackend):
        _call()


def test_merge_softmax_checks():
    a = SoftmaxState(torch.zeros(2, 3), torch.ones(2, 3), torch.zeros(2, 3, 4))
    b = SoftmaxState(torch.zeros(2, 4), torch.ones(2, 4), torch.zeros(2, 4, 4))
    with pytest.raises(ValueError, match="same queries"):
        aster_amd.merge_softmax(a, b)
    with pytest.raises(UnsupportedAttentionBackend):
        aster_amd.merge_softmax(a, a)
    s = SoftmaxState(torch.tensor([[0.0, -float("inf")]]), torch.tensor([[2.0, 0.0]]),
                     torch.tensor([[[4.0, 2.0], [0.0, 0.0]]]).reshape(1, 2, 2))
    # output() normalises as the reference does; a zero mass gives zeros
    out = SoftmaxState(s.maximum[None, None], s.mass[None, None], s.weighted[None, None]).output()
    assert out.shape == (1, 1, 2, 2)
    assert torch.equal(out[0, 0], torch.tensor([[2.0, 1.0], [0.0, 0.0]]))
