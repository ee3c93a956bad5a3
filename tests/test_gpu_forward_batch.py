"""The reference runner's entry point on the hip_int8_paged backend:
``PagedAttentionRunner(model, policy_artifact_id=..., backend="hip_int8_paged")`` and
``forward_batch(sequences, chunks, *, return_all_logits, padding_masks)``
(paged_attention.py:22-50, 110-230) over a Llama/Qwen-shaped test model with GQA, a
sliding-window layer and q/k norms, through prefill chunks, decode steps, padding, a
fork with copy-on-write and groups of different lengths.

fp32 model: a CPU rendering of the reference's row loop over the same weights (torch
fp32 model parts, the oracle's quantize-then-attend per row over quantized history
pages plus the chunk block) computes its own hidden states, queries, attention and
logits over the codes of the K/V values the GPU run produced (OracleLoop explains
why the codes are shared); every layer's attention and the logits match at the
north_star tolerance. Fed with the GPU run's q/k/v, the oracle's row loop gives each
layer's attention to the same tolerance and a quantized history that the pool's
pages equal bit for bit after every step.
bf16 model: the fed check only (the model parts in bf16 round differently on the
two sides)."""

import copy

import numpy as np
import pytest
import torch

from aster_amd import KVQuantization, UnsupportedAttentionBackend
from aster_amd.paged_pool import CacheCapacityError, StateError
from aster_amd.runner import PagedAttentionRunner
from tests.gpu_util import assert_attention_close
from tests.llama_like import LlamaLike
from tests.oracle_rows import OracleRows, check_pool_matches_oracle

pytestmark = pytest.mark.gpu


class Recorder:
    """Forward hooks: each layer's q (after norm and RoPE), k, v (packed [T, H, D]) and
    attention output (the o_proj input), per forward call."""

    def __init__(self, model):
        self.calls = []
        for index, layer in enumerate(model.model.layers):
            attention = layer.self_attn
            rope = attention.rope
            attention.rope = _RopeTap(rope, self, index)
            attention.v_proj.register_forward_hook(self._hook(index, "v"))
            attention.o_proj.register_forward_hook(self._hook(index, "o", inputs=True))

    def _hook(self, index, name, inputs=False):
        def hook(module, args, output):
            x = args[0] if inputs else output
            self.calls[-1].setdefault(index, {})[name] = x.detach().clone()
        return hook

    def begin(self):
        self.calls.append({})


class _RopeTap(torch.nn.Module):
    """Wraps a layer's rope: its first call per layer gives q, the second k."""

    def __init__(self, rope, recorder, index):
        super().__init__()
        self.rope, self.recorder, self.index = rope, recorder, index

    def forward(self, x, positions):
        y = self.rope(x, positions)
        slot = self.recorder.calls[-1].setdefault(self.index, {})
        slot["k" if "q" in slot else "q"] = y.detach().clone()
        return y


def _pack(x):
    """[B, H, T, D] -> packed [B*T, H, D] numpy (rows in batch order)."""
    b, h, t, d = x.shape
    return x.transpose(1, 2).reshape(b * t, h, d).float().cpu().numpy()


class OracleLoop:
    """The reference's forward_batch (paged_attention.py:144-230) on the CPU for an
    fp32 model: torch for the model parts, OracleRows for the paged attention.

    ``shared_kv`` (per layer, the step's K/V as the GPU run produced them) makes the
    oracle quantize those values instead of its own: quantization is a step function,
    and after layer 0 the two sides' fp32 values differ in the last bits, which moves
    a few codes by one quantization step (~1 % of a row's range); with the codes
    shared (their bit-exactness is checked on the pool), everything else -- hidden
    states, queries, attention, logits -- is computed independently here and differs
    only by rounding."""

    def __init__(self, model):
        self.model = copy.deepcopy(model).float().cpu().eval()
        self.rows = OracleRows(len(self.model.model.layers))

    @torch.no_grad()
    def forward(self, keys, start, chunks, padding=None, shared_kv=None):
        batch, count = len(chunks), len(chunks[0])
        ids = torch.tensor(chunks)
        positions = torch.arange(start, start + count).expand(batch, -1)
        hidden = self.model.model.embed_tokens(ids)
        rows = [(key, start, count) for key in keys]
        pads = None if padding is None else [np.asarray(p, bool) for p in padding]
        attended = []
        self.states = []  # each layer's input, then the normed output
        for index, layer in enumerate(self.model.model.layers):
            self.states.append(hidden)
            attention = layer.self_attn
            normalized = layer.input_layernorm(hidden)

            def split(value, heads):
                return value.reshape(batch, count, heads, attention.head_dim).transpose(1, 2)

            q = attention.rope(attention.q_norm(split(attention.q_proj(normalized),
                                                      attention.num_heads)), positions)
            k = attention.rope(attention.k_norm(split(attention.k_proj(normalized),
                                                      attention.num_kv_heads)), positions)
            v = split(attention.v_proj(normalized), attention.num_kv_heads)
            kp, vp = shared_kv[index] if shared_kv is not None else (_pack(k), _pack(v))
            out = self.rows.attend(index, rows, _pack(q), kp, vp, attention.scale, pads,
                                   window=attention.window)
            attended.append(out)
            result = torch.from_numpy(out).reshape(batch, count, -1)
            hidden = hidden + attention.o_proj(result)
            hidden = hidden + layer.mlp(layer.post_attention_layernorm(hidden))
        normed = self.model.model.norm(hidden)
        self.states.append(normed)
        logits = self.model.lm_head(normed)
        return logits, attended


def _tokens(rng, vocab, batch, count):
    return [rng.integers(0, vocab, count).tolist() for _ in range(batch)]


def test_forward_batch_matches_reference_row_loop_fp32(device):
    model = LlamaLike(seed=1).to(device)
    runner = PagedAttentionRunner(model, policy_artifact_id="policy-a", backend="hip_int8_paged",
                                  max_blocks=64)
    recorder = Recorder(runner.model)
    oracle = OracleLoop(model)
    fed = OracleRows(2)
    pool = runner.pool
    assert pool.cache is None  # the arena is allocated at the first step
    rng = np.random.default_rng(3)
    vocab = model.config.vocab_size
    seqs = [pool.create("policy-a") for _ in range(3)]
    keys = ["a", "b", "c"]

    def step(seqs, keys, chunks, padding=None, all_logits=False):
        start, count = seqs[0].length, len(chunks[0])
        recorder.begin()
        got = runner.forward_batch(seqs, chunks, return_all_logits=all_logits,
                                   padding_masks=padding)
        calls = recorder.calls[-1]
        shared = {i: (_pack(c["k"]), _pack(c["v"].reshape(len(seqs), count, 2, 64)
                                           .transpose(1, 2))) for i, c in calls.items()}
        want, attended = oracle.forward(keys, start, chunks, padding, shared_kv=shared)
        pads = None if padding is None else [np.asarray(p, bool) for p in padding]
        for index, out in enumerate(attended):
            o = calls[index]["o"].reshape(out.shape)
            assert_attention_close(o, out)
            attention = runner.model.model.layers[index].self_attn
            assert_attention_close(o, fed.attend(index, [(k, start, count) for k in keys],
                                                 _pack(calls[index]["q"]), *shared[index],
                                                 attention.scale, pads,
                                                 window=attention.window))
        for row, logits in enumerate(got):
            assert logits.dtype == torch.float32 and logits.device.type == "cpu"
            expect = want[row] if all_logits else want[row, -1]
            assert_attention_close(logits, expect)
        return got

    # prefill: one 37-token chunk per row, a padded row among them (return_all_logits)
    pad = np.ones((3, 37), bool)
    pad[1, 5:9] = False
    pad[2, ::3] = False
    got = step(seqs, keys, _tokens(rng, vocab, 3, 37), pad.tolist(), all_logits=True)
    assert got[0].shape == (37, vocab) and runner.attention_work.backend == "hip_int8_paged"
    assert pool.cache is not None and pool.cache.num_layers == 2
    for _ in range(3):  # decode steps
        got = step(seqs, keys, _tokens(rng, vocab, 3, 1))
        assert got[0].shape == (vocab,)
    # fork row 0 (same length): both extend the shared partial tail page (COW)
    fork = pool.fork(seqs[0])
    oracle.rows.fork("a", "d")
    fed.fork("a", "d")
    tail = seqs[0].pages[-1]
    step([seqs[0], fork], ["a", "d"], _tokens(rng, vocab, 2, 3))
    assert seqs[0].pages[-1] != tail and fork.pages[-1] != tail
    # a group of another length in its own call (rows grouped by the scheduler)
    step([seqs[1], seqs[2]], ["b", "c"], _tokens(rng, vocab, 2, 2))
    for s, k in zip(seqs + [fork], keys + ["d"]):
        check_pool_matches_oracle(pool, fed, s, k)
    assert runner.forward_calls == 6 and runner.input_tokens_computed == 3 * 37 + 9 + 6 + 4
    # the layout is locked: an append with another input dtype is refused (state.py:297-300)
    seq = pool.create("policy-a")
    bad = tuple((torch.zeros(1, 2, 3, 64, device=device, dtype=torch.bfloat16),) * 2
                for _ in range(2))
    with pytest.raises(StateError, match="layout"):
        pool.append_delta(seq, bad)
    for s in seqs + [fork]:
        pool.release(s)
    assert pool.used_blocks == 0


def test_forward_batch_bf16_layers_match_oracle(device):
    model = LlamaLike(seed=2, heads=16, kv_heads=4, head_dim=128, hidden=512, windows=(None, 40),
                      qk_norm=False).to(device, torch.bfloat16)
    runner = PagedAttentionRunner(model, policy_artifact_id="policy-b", backend="hip_int8_paged",
                                  max_blocks=128)
    recorder = Recorder(runner.model)
    rows = OracleRows(2)
    pool = runner.pool
    rng = np.random.default_rng(4)
    vocab = model.config.vocab_size
    seqs = [pool.create("policy-b") for _ in range(4)]
    keys = list("wxyz")
    for count in (70, 1, 1, 17, 1):
        start = seqs[0].length
        recorder.begin()
        logits = runner.forward_batch(seqs, _tokens(rng, vocab, 4, count))
        assert all(torch.isfinite(x).all() for x in logits)
        for index, layer in enumerate(runner.model.model.layers):
            rec = recorder.calls[-1][index]
            v = rec["v"].reshape(4, count, 4, 128).transpose(1, 2)
            want = rows.attend(index, [(k, start, count) for k in keys], _pack(rec["q"]),
                               _pack(rec["k"]), _pack(v), layer.self_attn.scale,
                               window=layer.self_attn.window)
            assert_attention_close(rec["o"].reshape(want.shape), want)
    for s, k in zip(seqs, keys):
        check_pool_matches_oracle(pool, rows, s, k)


def test_forward_batch_argument_checks_and_rollback(device):
    model = LlamaLike(seed=3).to(device)
    runner = PagedAttentionRunner(model, policy_artifact_id="p", backend="hip_int8_paged",
                                  max_blocks=8, kv_quantization=KVQuantization("fp8_e4m3fn"))
    pool = runner.pool
    a, b = pool.create("p"), pool.create("p")
    with pytest.raises(ValueError, match="distinct"):
        runner.forward_batch([a, a], [[1], [2]])
    with pytest.raises(ValueError, match="group matching"):
        runner.forward_batch([a, b], [[1, 2], [3]])
    with pytest.raises(ValueError, match="vocabulary"):
        runner.forward_batch([a], [[10 ** 6]])
    with pytest.raises(ValueError, match="binary"):
        runner.forward_batch([a], [[1, 2]], padding_masks=[[1, 2]])
    with pytest.raises(StateError, match="security"):
        runner.forward_batch([a, pool.create("q")], [[1], [2]])
    runner.forward_batch([a, b], [[1, 2, 3]] * 2)
    used = pool.used_blocks
    # 8 blocks of 16 tokens: 3 + 40 tokens per row needs 3 pages each -> nothing committed
    with pytest.raises(CacheCapacityError):
        runner.forward_batch([a, b], [[1] * 200] * 2)
    assert pool.used_blocks == used and a.length == b.length == 3
    with pytest.raises(ValueError, match="backend"):
        PagedAttentionRunner(model, policy_artifact_id="p", backend="torch_online_paged")
    with pytest.raises(ValueError, match="fallback"):
        PagedAttentionRunner(model, policy_artifact_id="p", backend="hip_int8_paged",
                             attention_fallback="torch_online")
    with pytest.raises(UnsupportedAttentionBackend):
        PagedAttentionRunner(model, policy_artifact_id="p", backend="hip_int8_paged",
                             block_size=32)


def test_forward_feature_batch_returns_the_requested_hidden_states(device):
    """forward_feature_batch (src/aster/inference/runner.py:72-83, 124-145): every row's
    logits for all chunk tokens with the requested hidden states concatenated along the
    hidden axis (index 0 the embeddings, i the input of layer i, num_layers the normed
    output), against the oracle's row loop; an index past the last state raises the
    reference's StateError and appends nothing."""
    model = LlamaLike(seed=5).to(device)
    runner = PagedAttentionRunner(model, policy_artifact_id="f", backend="hip_int8_paged",
                                  max_blocks=32)
    recorder = Recorder(runner.model)
    oracle = OracleLoop(model)
    pool = runner.pool
    rng = np.random.default_rng(6)
    vocab, hidden = model.config.vocab_size, model.model.embed_tokens.embedding_dim
    seqs = [pool.create("f") for _ in range(2)]
    for count, picks in ((19, (0, 1, 2)), (1, (2,)), (4, (1, 0))):
        start = seqs[0].length
        chunks = _tokens(rng, vocab, 2, count)
        recorder.begin()
        got = runner.forward_feature_batch(seqs, chunks, hidden_state_indices=picks)
        calls = recorder.calls[-1]
        shared = {i: (_pack(c["k"]), _pack(c["v"].reshape(2, count, 2, 64).transpose(1, 2)))
                  for i, c in calls.items()}
        want, _ = oracle.forward(["a", "b"], start, chunks, shared_kv=shared)
        expect = torch.cat([oracle.states[i] for i in picks], -1)
        assert len(got) == 2
        for row, (logits, feature) in enumerate(got):
            assert logits.shape == (count, vocab) and logits.device.type == "cpu"
            assert feature.shape == (count, hidden * len(picks))
            assert feature.device == torch.device(device)
            assert_attention_close(logits, want[row])
            assert_attention_close(feature, expect[row])
    length = seqs[0].length
    with pytest.raises(StateError, match="aligned target features"):
        runner.forward_feature_batch(seqs, _tokens(rng, vocab, 2, 1), hidden_state_indices=(3,))
    assert seqs[0].length == seqs[1].length == length
    with pytest.raises(ValueError, match="nonnegative"):
        runner.forward_feature_batch(seqs, _tokens(rng, vocab, 2, 1), hidden_state_indices=(-1,))
    with pytest.raises(ValueError, match="nonnegative"):
        runner.forward_feature_batch(seqs, _tokens(rng, vocab, 2, 1), hidden_state_indices=())
