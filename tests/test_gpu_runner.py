"""Runner integration of the hip_int8_paged backend: a toy GQA decoder steps through
PagedAttentionStep over the arena-backed pool (ragged prefill chunks, decode,
fork + copy-on-write, a mixed step, an aborted step, a step with non-finite input). At every layer the HIP
attention output is checked against the oracle's rendering of the reference's
forward_batch row loop (paged_attention.py:168-215): the row's quantized history
pages plus the chunk's own quantized K/V as one more block, causal positions,
dequantize-then-attend; and after every step the pool's pages equal the oracle's
quantized history bit for bit."""

import numpy as np
import pytest
import torch

from aster_amd import KernelWork, PagedKVCache
from aster_amd.paged_pool import PagedStatePool
from aster_amd.runner import PagedAttentionStep, pack_rows, unpack_rows
from tests.gpu_util import assert_attention_close
from tests.oracle_rows import OracleRows, check_pool_matches_oracle
from tests.tiny_decoder import TinyDecoder

pytestmark = pytest.mark.gpu


def run_step(model, pool, oracle, seqs, keys, chunks, work, padding=None):
    counts = [len(c) for c in chunks]
    ids = torch.tensor([t for c in chunks for t in c], device=pool.cache.device)
    with PagedAttentionStep(pool, seqs, counts, work=work, padding=padding) as step:
        pos = torch.cat([torch.arange(p, p + n) for p, n in zip(step.positions, counts)])
        rows = list(zip(keys, step.positions, counts))

        def attend(layer, q, k, v):
            out = step.attend(layer, q, k, v, scale=model.scale)
            want = oracle.attend(layer, rows, q.cpu().numpy(), k.cpu().numpy(),
                                 v.cpu().numpy(), model.scale, padding)
            assert_attention_close(out, want)
            return out

        logits = model.forward(ids, pos.to(ids.device), attend)
    return logits


def test_runner_steps_match_reference_row_loop(device):
    model = TinyDecoder(device)
    pool = PagedStatePool(PagedKVCache(num_blocks=48, num_layers=model.layers,
                                       num_kv_heads=model.hkv, head_dim=model.d, device=device))
    oracle = OracleRows(model.layers)
    rng = np.random.default_rng(0)
    seqs = [pool.create("tenant") for _ in range(3)]
    keys = ["a", "b", "c"]
    work = KernelWork()

    def tokens(n):
        return rng.integers(0, model.vocab, n).tolist()

    # 1. ragged prefill chunks
    run_step(model, pool, oracle, seqs, keys, [tokens(20), tokens(7), tokens(33)], work)
    assert [s.length for s in seqs] == [20, 7, 33] and work.backend == "hip_int8_paged"
    # 2. one decode token each
    logits = run_step(model, pool, oracle, seqs, keys, [tokens(1)] * 3, work)
    assert logits.shape == (3, model.vocab) and torch.isfinite(logits).all()
    # 3. fork seq 0 and run a mixed step: both the fork and its parent extend the
    #    shared partial tail page, so each gets a private copy
    fork = pool.fork(seqs[0])
    oracle.fork("a", "d")
    tail = seqs[0].pages[-1]
    run_step(model, pool, oracle, [seqs[0], seqs[1], fork], ["a", "b", "d"],
             [tokens(1), tokens(5), tokens(2)], work)
    assert seqs[0].pages[-1] != tail and fork.pages[-1] != tail
    assert [seqs[0].length, seqs[1].length, fork.length] == [22, 13, 23]
    for s, k in zip(seqs + [fork], keys + ["d"]):
        check_pool_matches_oracle(pool, oracle, s, k)
    # 4. chunks with padding tokens (forward_batch padding_masks, paged_attention.py:137-143):
    #    appended, attended by no query, now or in the decode step after
    pads = [rng.random(n) > 0.3 for n in (6, 1, 9)]
    pads[2][:3] = False
    run_step(model, pool, oracle, seqs, keys, [tokens(6), tokens(1), tokens(9)], work,
             padding=[torch.tensor(p) for p in pads])
    assert pool.cache.has_padding
    run_step(model, pool, oracle, seqs, keys, [tokens(1)] * 3, work)
    for s, k in zip(seqs + [fork], keys + ["d"]):
        check_pool_matches_oracle(pool, oracle, s, k)
    with pytest.raises(ValueError, match="binary"):
        PagedAttentionStep(pool, seqs, [2, 2, 2], padding=[[1, 2], [1, 1], [1, 1]])
    # 5. a step that fails midway commits nothing
    used, lengths = pool.used_blocks, [s.length for s in seqs]
    with pytest.raises(RuntimeError, match="layer failed"):
        with PagedAttentionStep(pool, seqs, [16, 16, 16]) as step:
            raise RuntimeError("layer failed")
    assert pool.used_blocks == used and [s.length for s in seqs] == lengths
    # 6. a chunk holding a non-finite key: the step appends in one launch into its
    #    reserved slots, the flag raises the reference's error at commit and every
    #    reservation is rolled back, so the pool is as before (kv_quantization.py:77-81
    #    raises before PagedStatePool.append_delta changes anything)
    with pytest.raises(ValueError, match="finite"):
        with PagedAttentionStep(pool, seqs, [1, 4, 1]) as step:
            key = torch.randn(6, model.hkv, model.d, device=device)
            key[3, 0, 5] = float("nan")
            q = torch.randn(6, model.hq, model.d, device=device)
            step.attend(0, q, key, torch.randn_like(key), scale=model.scale)
    assert pool.used_blocks == used and [s.length for s in seqs] == lengths
    for s, k in zip(seqs + [fork], keys + ["d"]):
        check_pool_matches_oracle(pool, oracle, s, k)
    run_step(model, pool, oracle, seqs, keys, [tokens(1)] * 3, work)  # the flag was cleared
    for s in seqs + [fork]:
        pool.release(s)
    assert pool.used_blocks == 0


def test_pack_unpack_reference_layout(device):
    x = torch.randn(3, 4, 5, 8, device=device)
    counts = [5, 2, 4]
    packed = pack_rows(x, counts)
    assert packed.shape == (11, 4, 8)
    back = unpack_rows(packed, counts, 5)
    for b, n in enumerate(counts):
        assert torch.equal(back[b, :, :n], x[b, :, :n])
        assert (back[b, :, n:] == 0).all()


def test_bf16_decode_step_with_nonfinite_key_rolls_back(device):
    """A bf16 decode step appends inside the planned attention launch; a non-finite
    key raises the reference's error at commit and rolls every reservation back: the
    pool's pages equal those before the step, token for token."""
    pool = PagedStatePool(PagedKVCache(num_blocks=64, num_layers=1, num_kv_heads=2,
                                       head_dim=128, device=device))
    seqs = [pool.create("tenant") for _ in range(3)]
    gen = torch.Generator(device=device).manual_seed(7)

    def rows(n, heads):
        return torch.randn(n, heads, 128, generator=gen, device=device).to(torch.bfloat16)

    with PagedAttentionStep(pool, seqs, [37, 5, 20]) as step:  # a prefill step
        step.attend(0, rows(62, 8), rows(62, 2), rows(62, 2), scale=128 ** -0.5)
    before = [pool.materialize(s) for s in seqs]
    used = pool.used_blocks
    key = rows(3, 2)
    key[1, 1, 9] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        with PagedAttentionStep(pool, seqs, [1, 1, 1]) as step:
            assert step.attend(0, rows(3, 8), key, rows(3, 2),
                               scale=128 ** -0.5).shape == (3, 8, 128)
    assert pool.used_blocks == used and [s.length for s in seqs] == [37, 5, 20]
    for s, old in zip(seqs, before):
        for a, b in zip(pool.materialize(s), old):
            for x, y in zip(a, b):
                assert torch.equal(x, y)
    # a clean decode step then commits (the flag was cleared)
    with PagedAttentionStep(pool, seqs, [1, 1, 1]) as step:
        step.attend(0, rows(3, 8), rows(3, 2), rows(3, 2), scale=128 ** -0.5)
    assert [s.length for s in seqs] == [38, 6, 21]
