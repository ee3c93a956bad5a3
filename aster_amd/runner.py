"""The attention part of a paged forward step on the ``hip_int8_paged`` backend.

``PagedAttentionRunner.forward_batch`` (src/aster/inference/paged_attention.py:110-230)
takes read leases on every row's pages, and per layer runs one ``online_attention``
per row over the row's pages plus the chunk's own (quantized) K/V, appending the
chunk to the pool only after the step (:226-229). ``PagedAttentionStep`` replaces
that row loop:

  * on entry it reserves the step's slots in the pool for every row
    (transactionally: all rows or none) and builds one block table over the
    reserved pages, with ``query_start_loc`` packing ragged chunk lengths;
  * per layer, ``attend`` quantize-appends the chunk K/V of all rows into their
    slots in one launch and runs one ragged attention launch (decode rows on the
    decode kernels, chunk rows on the prefill kernel) over history + chunk,
    causal within the chunk, exactly the keys the reference's per-row call sees;
    a planned decode step with bf16/fp16 rows (head dims 128, 256) appends inside
    the attention launch;
  * on exit it checks the device error flag and commits every reservation, or
    rolls all of them back if the step raised.

Row lengths need not match (the reference groups equal ``start``/``count`` per
call, :118-123). Chunk padding (``forward_batch(padding_masks=...)``, :137-143) is
written once per step into the reserved slots' key bytes: a padding token is
appended like any other but attended by no query, in this step or later, as the
reference's padding leaf does (:181, :190, :228).
"""

from __future__ import annotations

import copy
import time

import numpy as np
import torch

from .attention_backend import BACKEND, KernelWork, UnsupportedAttentionBackend
from .kv_quantization import KVQuantization
from .paged_pool import KVStateCodec, PagedStatePool, StateError
from .prefix_plan import plan_prefix_packs


def pack_rows(x, counts):
    """Reference layout ``[B, H, Q, D]`` (rows padded to Q) -> packed ``[sum(counts), H, D]``."""
    if x.ndim != 4 or x.shape[0] != len(counts):
        raise ValueError("expected [batch, heads, tokens, head_dim] rows")
    rows = [x[b, :, :n].transpose(0, 1) for b, n in enumerate(counts)]
    return torch.cat(rows, 0).contiguous() if rows else x.new_empty((0, x.shape[1], x.shape[3]))


def unpack_rows(y, counts, width=None):
    """Packed ``[sum(counts), H, D]`` -> ``[B, H, width, D]`` (zero-padded rows)."""
    width = width or max(counts)
    out = y.new_zeros((len(counts), y.shape[1], width, y.shape[2]))
    cursor = 0
    for b, n in enumerate(counts):
        out[b, :, :n] = y[cursor : cursor + n].transpose(0, 1)
        cursor += n
    return out


def _device_ints(values, dtype, device):
    """A host list of step metadata as a device vector (an async upload)."""
    return torch.tensor(values, dtype=dtype).to(device, non_blocking=True)


def _padding_vector(padding, counts):
    """Chunk padding as a host bool vector packed like the step's tokens: one 0/1
    sequence per row (``len == counts[b]``) or a batch-by-token matrix whose row ``b``
    starts with the row's ``counts[b]`` tokens (paged_attention.py:137-143)."""
    rows = []
    if isinstance(padding, (list, tuple)):
        if len(padding) != len(counts):
            raise ValueError("Chunk padding must be a binary batch-by-token matrix")
        for row, n in zip(padding, counts):
            row = torch.as_tensor(row).cpu()
            if row.ndim != 1 or row.shape[0] != n:
                raise ValueError("Chunk padding must be a binary batch-by-token matrix")
            rows.append(row)
    else:
        matrix = torch.as_tensor(padding).cpu()
        if matrix.ndim != 2 or matrix.shape[0] != len(counts) or matrix.shape[1] < max(counts):
            raise ValueError("Chunk padding must be a binary batch-by-token matrix")
        rows = [matrix[b, :n] for b, n in enumerate(counts)]
    packed = torch.cat(rows)
    if not ((packed == 0) | (packed == 1)).all():
        raise ValueError("Chunk padding must be a binary batch-by-token matrix")
    return packed.bool()


class PagedAttentionStep:
    """One step of ``counts[b]`` new tokens for each sequence ``b`` of a batch."""

    def __init__(self, pool, sequences, counts, *, padding=None, work=None,
                 partition_tokens=0):
        if not sequences or len(sequences) != len(counts) or \
                len({id(s) for s in sequences}) != len(sequences):
            raise ValueError("Need a nonempty batch of distinct sequences and aligned chunks")
        if any(type(n) is not int or n < 1 for n in counts):
            raise ValueError("Every row needs at least one new token")
        if len({s.identity for s in sequences}) != 1:
            raise StateError("A projection batch cannot cross cache security domains")
        valid = None if padding is None else _padding_vector(padding, counts)
        self.pool, self.counts = pool, list(counts)
        self.work = work if work is not None else KernelWork()
        self.partition_tokens = partition_tokens
        self.reservations = []
        self._tables = None
        self._open = False
        # every reservation and the read leases are undone if anything below raises
        try:
            for sequence, n in zip(sequences, counts):
                self.reservations.append(pool.reserve(sequence, n))
            cache = pool.cache
            device = cache.device
            tables = pool.block_tables(self.reservations)
            self.block_tables, self.context_lens = tables.__enter__()
            self._tables = tables
            starts = [0]
            for n in counts:
                starts.append(starts[-1] + n)
            self.num_tokens = starts[-1]
            self.query_start_loc = _device_ints(starts, torch.int32, device)
            self.positions = [r.start for r in self.reservations]
            self.max_query_len = max(counts)
            self.max_context_len = max(r.length for r in self.reservations)
            slots = [s for r in self.reservations for s in r.slots]
            self.slot_mapping = _device_ints(slots, torch.int64, device)
            cache.write_key_valid(self.slot_mapping,
                                  None if valid is None else valid.to(device, non_blocking=True))
            # decode steps: the rows' page lists, for prefix packs (planned per query-head
            # count at the first attend)
            self._pages = ([[ref.index for ref in r.pages] for r in self.reservations]
                           if len(counts) > 1 and self.max_query_len == 1 else None)
            self._packs = {}
            self._plans = {}
        except BaseException:
            if self._tables is not None:
                self._tables.__exit__(None, None, None)
            for r in self.reservations:
                pool.abort(r)
            raise
        self._open = True

    def attend(self, layer, query, key, value, *, scale=None, window=None, out=None):
        """Append this layer's chunk K/V and attend. ``query`` ``[T, Hq, D]`` and
        ``key``/``value`` ``[T, Hkv, D]`` packed by row in batch order (``pack_rows``
        converts the reference's ``[B, H, Q, D]``). Returns ``[T, Hq, D]`` in the
        query dtype."""
        if not self._open:
            raise StateError("Step already committed or aborted")
        if query.shape[0] != self.num_tokens or key.shape[0] != self.num_tokens:
            raise ValueError("query/key rows must match the step's tokens")
        cache = self.pool.cache
        ws_work = self.work
        plan = self._decode_plan(query, window) if self.partition_tokens == 0 else None
        if plan is not None:
            # decode rows on the host schedule (one per step and shape); rows aliasing
            # shared prefix pages read them once per prefix tile. bf16/fp16 rows are
            # appended by the decode itself (one launch), into the step's reserved slots
            fused = (cache.decode_appends(query.dtype) and key.dtype == query.dtype
                     and value.dtype == query.dtype)
            if not fused:
                cache.append(layer, key, value, self.slot_mapping, reserved=True)
            return cache.paged_attention(
                layer, query, self.block_tables, self.context_lens,
                max_context_len=self.max_context_len, scale=scale, window=window, out=out,
                work=ws_work, decode_plan=plan,
                append=(key, value, self.slot_mapping) if fused else None)
        # the step's slots are reserved and rolled back if the step is flagged
        cache.append(layer, key, value, self.slot_mapping, reserved=True)
        packs = (self._prefix_packs(query.shape[1])
                 if window is None and self.partition_tokens == 0 else None)
        if packs is not None:  # rows aliasing shared prefix pages read them once per pack
            return cache.paged_attention(
                layer, query, self.block_tables, self.context_lens,
                max_context_len=self.max_context_len, scale=scale, out=out, work=ws_work,
                partition_tokens=0, prefix_packs=packs)
        return cache.paged_attention(
            layer, query, self.block_tables, self.context_lens,
            max_context_len=self.max_context_len, scale=scale, window=window,
            partition_tokens=self.partition_tokens, query_start_loc=self.query_start_loc,
            max_query_len=self.max_query_len, causal=True, out=out, work=ws_work)

    def _host_tables(self):
        width = max(len(p) for p in self._pages)
        tables = np.full((len(self._pages), width), -1, np.int64)
        for row, pages in enumerate(self._pages):
            tables[row, : len(pages)] = pages
        return tables, [r.length for r in self.reservations]

    def _decode_plan(self, query, window):
        """The step's decode schedule for this query shape and window (built at the first
        layer that asks, reused by the others), or None where the planned kernel does
        not serve the step (a single row; fp32 queries over FP8 codes)."""
        cache = self.pool.cache
        if self._pages is None or not (query.dtype in (torch.bfloat16, torch.float16) or (
                query.dtype == torch.float32 and cache.code_format == 0)):
            return None  # fp32 queries: the planned kernel takes them over int8 codes
        key = (query.shape[1], query.dtype, window)
        if key not in self._plans:
            from .decode_plan import plan_decode

            cache = self.pool.cache
            tables, lens = self._host_tables()
            self._plans[key] = plan_decode(
                tables, lens, num_q_heads=query.shape[1], num_kv_heads=cache.num_kv_heads,
                head_dim=cache.head_dim, q_dtype=query.dtype, device=cache.device,
                code_format=cache.code_format, window=window)
        return self._plans[key]

    def _prefix_packs(self, num_q_heads):
        if self._pages is None:
            return None
        if num_q_heads not in self._packs:
            tables, lens = self._host_tables()
            cache = self.pool.cache
            self._packs[num_q_heads] = plan_prefix_packs(
                tables, lens, num_q_heads, cache.num_kv_heads, device=cache.device,
                block_size=cache.block_size)
        return self._packs[num_q_heads]

    def commit(self):
        """Wait for the device, raise any flagged error (then nothing is committed),
        release the read leases and publish every row's tokens."""
        if not self._open:
            raise StateError("Step already committed or aborted")
        try:
            torch.cuda.synchronize(self.pool.cache.device)
            self.pool.cache.raise_errors()
        except BaseException:
            self.abort()
            raise
        self._close()
        for r in self.reservations:
            self.pool.commit(r)
        self.work.backend, self.work.fallback_reason = BACKEND, None

    def abort(self):
        if not self._open:
            return
        torch.cuda.synchronize(self.pool.cache.device)
        self._close()
        for r in self.reservations:
            self.pool.abort(r)

    def _close(self):
        self._open = False
        self._tables.__exit__(None, None, None)

    def __enter__(self):
        return self

    def __exit__(self, kind, error, trace):
        if kind is None:
            self.commit()
        else:
            self.abort()
        return False


_ATTENTION_PARTS = ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm", "rope",
                    "num_heads", "num_kv_heads", "head_dim", "window", "scale")
_LAYER_PARTS = ("input_layernorm", "self_attn", "mlp", "post_attention_layernorm")


def _check_model(model):
    """The attributes the reference's paged forward loop touches
    (paged_attention.py:144-230), checked by shape instead of by the reference's model
    classes (paged_attention.py:56-70): a decoder ``model.model`` with ``embed_tokens``,
    ``layers`` and ``norm``, an ``lm_head``, a ``config`` with ``vocab_size`` and
    ``max_position_embeddings``, and per layer the GQA attention parts. Returns
    ``(num_layers, num_kv_heads, head_dim)``."""
    body = getattr(model, "model", None)
    if body is None or not all(hasattr(body, n) for n in ("embed_tokens", "layers", "norm")) \
            or not hasattr(model, "lm_head") or not hasattr(model, "config"):
        raise ValueError("Paged online runner needs a decoder with embed_tokens, layers, norm "
                         "and lm_head")
    config = model.config
    if not all(hasattr(config, n) for n in ("vocab_size", "max_position_embeddings")):
        raise ValueError("Paged online runner needs vocab_size and max_position_embeddings")
    if getattr(config, "attention_dropout", 0) != 0:
        raise ValueError("Unexpected attention/layer semantics or nonzero dropout")
    layers = list(body.layers)
    if not layers:
        raise ValueError("Paged online runner needs at least one decoder layer")
    shapes = set()
    for layer in layers:
        attention = getattr(layer, "self_attn", None)
        if not all(hasattr(layer, n) for n in _LAYER_PARTS) or \
                not all(hasattr(attention, n) for n in _ATTENTION_PARTS):
            raise ValueError("Unexpected attention/layer semantics or nonzero dropout")
        if attention.num_heads % attention.num_kv_heads:
            raise ValueError("Query heads must divide into KV groups")
        shapes.add((attention.num_kv_heads, attention.head_dim))
    if len(shapes) != 1:
        raise UnsupportedAttentionBackend("hip_int8_paged arenas hold one (kv heads, head dim) "
                                          "layout for every layer")
    hkv, dim = shapes.pop()
    return len(layers), hkv, dim


def bind_hip_backend(runner, model, *, policy_artifact_id, backend=BACKEND, tokenizer=None,
                     block_size=16, max_blocks=256, query_block_size=32, key_block_size=None,
                     chat_template=None, attention_fallback=None, kv_quantization=None,
                     partition_tokens=0):
    """Make ``runner`` a ``hip_int8_paged`` runner: the attributes the reference's
    ``PagedAttentionRunner.__init__`` sets (paged_attention.py:26-95 with
    ``ModelRunner.__init__``, runner.py:16-46), with this library's arena-backed pool.
    ``runner`` may be an instance of any class: the reference's own
    ``PagedAttentionRunner`` calls this from its constructor for
    ``backend="hip_int8_paged"``, so that callers which gate on the
    reference's class (``MultiLoRARunner``, adapters.py:47-50) accept it, and its
    ``forward_batch``/``forward_feature_batch`` then call :func:`hip_forward` /
    :func:`hip_forward_features` on it. The model is deep-copied once, as the
    reference does; everything later reads ``runner.model``, so module swaps on it
    (LoRA adapters) are seen by the step."""
    if backend != BACKEND:
        raise ValueError(f"Select explicit backend={BACKEND!r}")
    if attention_fallback is not None:
        raise ValueError("The hip_int8_paged backend takes no fallback: a configuration "
                         "it has no kernel for raises UnsupportedAttentionBackend")
    kv_quantization = KVQuantization("int8") if kv_quantization is None else kv_quantization
    if not isinstance(kv_quantization, KVQuantization):
        raise ValueError("An explicit immutable KVQuantization profile is required")
    key_block_size = 64 if key_block_size is None else key_block_size
    if any(type(v) is not int or v < 1 for v in (query_block_size, key_block_size)):
        raise ValueError("Attention tile sizes must be positive integers")
    if not isinstance(policy_artifact_id, str) or not policy_artifact_id:
        raise ValueError("An immutable policy identity is mandatory")
    runner.num_layers, runner.num_kv_heads, runner.head_dim = _check_model(model)
    shared = getattr(model, "_aster_shared_runtime_handles", ())
    runner.model = copy.deepcopy(model, {id(item): item for item in shared}).eval()
    runner.model.requires_grad_(False)
    runner.policy_artifact_id = policy_artifact_id
    runner.codec = KVStateCodec(kind="gqa_kv")
    runner.pool = PagedStatePool(block_size=block_size, max_blocks=max_blocks, codec=runner.codec,
                                 quantization=kv_quantization)
    runner.tokenizer, runner.chat_template = tokenizer, chat_template
    runner.device = next(runner.model.parameters(), torch.empty(0)).device
    runner.query_block_size, runner.key_block_size = query_block_size, key_block_size
    runner.backend = BACKEND
    runner.attention_fallback = None
    runner.partition_tokens = partition_tokens
    runner.attention_work = KernelWork(backend=BACKEND)
    runner.input_tokens_computed = 0
    runner.forward_calls = 0
    runner.model_execution_seconds = 0.0
    return runner


def _synchronize(device):
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def hip_forward(runner, sequences, chunks, *, return_all_logits=False, padding_masks=None,
                hidden_state_indices=None):
    """``PagedAttentionRunner.forward_batch`` (paged_attention.py:110-230) on a runner set
    up by :func:`bind_hip_backend`: the reference's argument checks and model walk, with
    every layer's attention as one ``PagedAttentionStep`` launch pair. With
    ``hidden_state_indices`` (see :func:`hip_forward_features`) every row's result is
    ``(logits, features)``."""
    if not sequences or len(sequences) != len(chunks) or \
            len({id(value) for value in sequences}) != len(sequences):
        raise ValueError("Need a nonempty batch of distinct sequences and aligned chunks")
    starts, counts = {s.length for s in sequences}, {len(chunk) for chunk in chunks}
    if len(starts) != 1 or len(counts) != 1 or min(counts) < 1:
        raise ValueError("Scheduler must group matching cached/chunk lengths")
    if len({s.identity for s in sequences}) != 1:
        raise StateError("A projection batch cannot cross cache security domains")
    model = runner.model
    config = model.config
    start, count, batch = next(iter(starts)), next(iter(counts)), len(sequences)
    if start + count > config.max_position_embeddings:
        raise ValueError("Sequence exceeds declared position support")
    if any(type(t) is not int or not 0 <= t < config.vocab_size for c in chunks for t in c):
        raise ValueError("Input token outside this immutable model vocabulary")
    device = runner.device
    ids = torch.tensor(chunks, device=device, dtype=torch.long)
    positions = torch.arange(start, start + count, device=device).expand(batch, -1)
    padding = None
    if padding_masks is not None:
        padding = torch.as_tensor(padding_masks).cpu()
        if padding.shape != ids.shape or not ((padding == 0) | (padding == 1)).all():
            raise ValueError("Chunk padding must be a binary batch-by-token matrix")
        padding = padding.bool()
    pool = runner.pool
    pool.bind_layout(num_layers=runner.num_layers, num_kv_heads=runner.num_kv_heads,
                     head_dim=runner.head_dim, device=device)
    layers = model.model.layers
    with torch.inference_mode():
        step = PagedAttentionStep(pool, sequences, [count] * batch, padding=padding,
                                  work=runner.attention_work,
                                  partition_tokens=runner.partition_tokens)
        try:
            _synchronize(device)
            started = time.monotonic()
            hidden = model.model.embed_tokens(ids)
            states = []  # each layer's input, then the normed output (hidden states)
            for index, layer in enumerate(layers):
                if hidden_state_indices is not None:
                    states.append(hidden)
                normalized = layer.input_layernorm(hidden)
                attention = layer.self_attn

                def split(value, heads):
                    return value.reshape(batch, count, heads, attention.head_dim).transpose(1, 2)

                query = attention.rope(attention.q_norm(
                    split(attention.q_proj(normalized), attention.num_heads)), positions)
                key = attention.rope(attention.k_norm(
                    split(attention.k_proj(normalized), attention.num_kv_heads)), positions)
                value = split(attention.v_proj(normalized), attention.num_kv_heads)
                if index == 0:  # the appended leaves' layout (state.py:285-300)
                    with pool._lock:
                        pool._lock_signature((runner.num_layers, runner.num_kv_heads,
                                              runner.head_dim, key.dtype))
                attended = step.attend(index, _packed(query), _packed(key), _packed(value),
                                       scale=attention.scale, window=attention.window)
                hidden = hidden + attention.o_proj(attended.reshape(batch, count, -1))
                hidden = hidden + layer.mlp(layer.post_attention_layernorm(hidden))
            normed = model.model.norm(hidden)
            logits = model.lm_head(normed)
            features = None
            if hidden_state_indices is not None:
                states.append(normed)
                if max(hidden_state_indices) >= len(states):
                    raise StateError("TokenPredictor did not return aligned target features")
                features = torch.cat([states[i] for i in hidden_state_indices], -1)
            step.commit()  # waits for the device, raises flagged errors, publishes
        except BaseException:
            step.abort()
            raise
        runner.model_execution_seconds += time.monotonic() - started
        runner.forward_calls += 1
        runner.input_tokens_computed += ids.numel()
    rows = [(row if return_all_logits else row[-1]).detach().float().cpu() for row in logits]
    if features is not None:
        return [(row, feature.detach()) for row, feature in zip(rows, features)]
    return rows


def hip_forward_features(runner, sequences, chunks, *, hidden_state_indices):
    """``ModelRunner.forward_feature_batch`` (src/aster/inference/runner.py:72-83,
    124-134, 143-145) through the paged step: every row's logits for all chunk tokens
    (CPU fp32) with the concatenation, along the hidden axis, of the requested hidden
    states (index i < num_layers: the input of layer i, index 0 the embeddings; index
    num_layers: the final normed output, as the reference decoder's
    ``output_hidden_states`` lists them, models/decoder.py:153-172), on the model's
    device. An index past the last state raises the reference's ``StateError`` and
    nothing is appended."""
    if not hidden_state_indices or any(type(i) is not int or i < 0 for i in hidden_state_indices):
        raise ValueError("Explicit nonnegative hidden-state indices are required")
    return hip_forward(runner, sequences, chunks, return_all_logits=True,
                       hidden_state_indices=tuple(hidden_state_indices))


class PagedAttentionRunner:
    """``PagedAttentionRunner`` (src/aster/inference/paged_attention.py:22-230) on the
    ``hip_int8_paged`` backend, with the reference's constructor and ``forward_batch``
    contract: the model's projections, norms, RoPE and MLP run as they are (PyTorch),
    and every layer's attention over the rows' pages plus the chunk is one
    quantize-append launch and one ragged attention launch on the HIP kernels
    (``PagedAttentionStep``). A thin class over :func:`bind_hip_backend`,
    :func:`hip_forward` and :func:`hip_forward_features`, which the reference's own class
    calls for ``backend="hip_int8_paged"``.

    Kept: the argument checks and exceptions of forward_batch (:110-143), read leases
    held until the device has finished (:144-148, :221), chunk K/V quantized before
    attention (the step writes them into reserved slots first, then attends over
    history + chunk: the same keys as the reference's extra quantized block,
    :185-192), key padding from ``padding_masks`` (:137-143, :181, :228), the chunk
    appended to the pool after the step (:226-229), CPU fp32 logits (:230),
    ``attention_work``, and the counters of ``ModelRunner`` (runner.py:44-46).
    Different: rows may not be committed one by one; the step commits all rows or, if
    anything raises, none (a full pool raises ``CacheCapacityError`` before any layer
    runs, not after). ``query_block_size``/``key_block_size`` are validated and kept
    but do not shape the kernels (their tiles are fixed: 16-token blocks, query tiles
    of 128 (token, head) columns). ``kv_quantization=None`` means the backend's INT8.
    """

    backend = BACKEND
    kind = "token_predictor"

    def __init__(self, model, *, policy_artifact_id, backend, **kwargs):
        bind_hip_backend(self, model, policy_artifact_id=policy_artifact_id, backend=backend,
                         **kwargs)

    @classmethod
    def from_artifact(cls, store, artifact_id, *, loader, tokenizer_loader=None, **kwargs):
        artifact = store.get(artifact_id, verify=True)
        tokenizer = tokenizer_loader(artifact.path) if tokenizer_loader else None
        return cls(loader(artifact.path), policy_artifact_id=artifact.id, tokenizer=tokenizer,
                   **kwargs)

    def forward_batch(self, sequences, chunks, *, return_all_logits=False, padding_masks=None):
        return hip_forward(self, sequences, chunks, return_all_logits=return_all_logits,
                           padding_masks=padding_masks)

    def forward_feature_batch(self, sequences, chunks, *, hidden_state_indices):
        return hip_forward_features(self, sequences, chunks,
                                    hidden_state_indices=hidden_state_indices)

    def decode(self, token_ids):
        if self.tokenizer is None:
            return " ".join(str(token) for token in token_ids)
        return self.tokenizer.decode(token_ids)

    def stream_text(self, token_ids, *, final=False):
        return self.decode(token_ids)


def _packed(x):
    """Reference layout ``[B, H, T, D]`` -> packed rows ``[B * T, H, D]`` (contiguous)."""
    batch, heads, tokens, dim = x.shape
    return x.transpose(1, 2).reshape(batch * tokens, heads, dim)
