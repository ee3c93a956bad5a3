"""The reference's forward_batch row loop (paged_attention.py:168-215) as test
infrastructure: per sequence and layer, the quantized history pages the reference
would hold, and each row's online attention over them plus the chunk's own quantized
K/V as one more block, through the oracle (dequantize-then-attend)."""

import numpy as np

from oracle import reference_cpu as ref


class OracleRows:
    """Per sequence and layer, the reference path's quantized history (host)."""

    def __init__(self, layers):
        self.layers = layers
        self.hist = {}  # (seq key, layer) -> (k codes/scales, v codes/scales) lists
        self.pad = {}   # seq key -> list of per-chunk bool padding leaves (True = real)

    def fork(self, src, dst):
        for layer in range(self.layers):
            self.hist[(dst, layer)] = [list(x) for x in self.hist.get((src, layer), ([], []))]
        self.pad[dst] = list(self.pad.get(src, []))

    def attend(self, layer, rows, q, k, v, scale, padding=None, window=None):
        """rows: list of (seq key, start, count) in packed order; q/k/v packed host arrays;
        padding: per row bool vector (True = real token) or None; window: the layer's
        sliding window (online_attention.py:183-184) or None."""
        outs, cursor = [], 0
        for r, (key, start, count) in enumerate(rows):
            pad = np.ones(count, bool) if padding is None else np.asarray(padding[r], bool)
            qs = q[cursor: cursor + count].transpose(1, 0, 2)[None]
            ks = k[cursor: cursor + count].transpose(1, 0, 2)[None]
            vs = v[cursor: cursor + count].transpose(1, 0, 2)[None]
            cursor += count
            hk, hv = self.hist.setdefault((key, layer), ([], []))
            qk, qv = ref.quantize_kv_int8(ks), ref.quantize_kv_int8(vs)
            pads = self.pad.setdefault(key, [])
            blocks = []
            if hk:
                blocks.append(ref.AttentionBlock(_cat(hk), _cat(hv), 0,
                                                 np.concatenate(pads[:len(hk)])[None]))
            blocks.append(ref.AttentionBlock(qk, qv, start, pad[None]))
            pos = np.arange(start, start + count)[None]
            out = ref.online_attention(qs, blocks, query_positions=pos, causal=True, scale=scale,
                                       window=window)
            outs.append(out[0].transpose(1, 0, 2))
            hk.append(qk), hv.append(qv)
            if layer == 0:
                pads.append(pad)
        return np.concatenate(outs, 0)


def _cat(parts):
    return ref.QuantizedKV(np.concatenate([p.values for p in parts], 2),
                           np.concatenate([p.scales for p in parts], 2))


def check_pool_matches_oracle(pool, oracle, seq, key):
    state = pool.materialize(seq)
    for layer, (k, v) in enumerate(state[:oracle.layers]):
        hk, hv = oracle.hist[(key, layer)]
        np.testing.assert_array_equal(k.cpu().numpy(), _cat(hk).dequantize())
        np.testing.assert_array_equal(v.cpu().numpy(), _cat(hv).dequantize())
    np.testing.assert_array_equal(state[-1][0][0, 0, :, 0].cpu().numpy(),
                                  np.concatenate(oracle.pad[key]))
