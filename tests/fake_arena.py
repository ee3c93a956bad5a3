"""A CPU stand-in for PagedKVCache with the same arena layout, used to test the
pool's host-side bookkeeping without a GPU. Appends quantize with the oracle
(test infrastructure only); block moves are plain tensor copies."""

import numpy as np
import torch

from aster_amd.kv_quantization import KVQuantization, QuantizedKV
from oracle import reference_cpu as ref


class FakeArena:
    def __init__(self, *, num_blocks, num_layers, num_kv_heads, head_dim, block_size=16):
        self.num_blocks, self.num_layers = num_blocks, num_layers
        self.num_kv_heads, self.head_dim, self.block_size = num_kv_heads, head_dim, block_size
        self.quantization = KVQuantization("int8")
        self.device = torch.device("cpu")
        self.codes = torch.zeros((num_blocks, num_layers, 2, num_kv_heads, block_size, head_dim),
                                 dtype=torch.int8)
        self.scales = torch.ones((num_blocks, num_layers, 2, num_kv_heads, block_size))
        self.key_valid = torch.ones((num_blocks, block_size), dtype=torch.uint8)
        self.has_padding = False
        self.flags = 0
        self.copies = []
        self.appends = 0

    @property
    def block_code_bytes(self):
        return self.codes[0].numel()

    @property
    def block_scale_bytes(self):
        return self.scales[0].numel() * 4

    def append(self, layer, key, value, slots):
        k, v = key.float().numpy(), value.float().numpy()
        if not (np.isfinite(k).all() and np.isfinite(v).all()):
            self.flags |= 1
            return
        self.appends += 1
        for kv, x in ((0, k), (1, v)):
            q = ref.quantize_kv_int8(x.transpose(1, 0, 2)[None])
            for t, slot in enumerate(slots.tolist()):
                b, o = divmod(slot, self.block_size)
                self.codes[b, layer, kv, :, o] = torch.from_numpy(q.values[0, :, t])
                self.scales[b, layer, kv, :, o] = torch.from_numpy(q.scales[0, :, t, 0])

    def write_key_valid(self, slots, valid=None):
        if valid is None and not self.has_padding:
            return
        self.has_padding = self.has_padding or valid is not None
        for t, slot in enumerate(slots.tolist()):
            b, o = divmod(slot, self.block_size)
            self.key_valid[b, o] = 1 if valid is None else int(bool(valid[t]))

    def code_view(self, raw):
        return raw.view(self.quantization.dtype)

    def padding_leaf(self, block):
        return self.key_valid[block].view(torch.bool)[None, None, :, None]

    def raise_errors(self):
        flags, self.flags = self.flags, 0
        if flags:
            raise ValueError("Quantized KV requires finite floating input")

    def copy_blocks(self, src, dst, *, stream=None):
        self.copies.append((list(src), list(dst)))
        for s, d in zip(src, dst):
            self.codes[d] = self.codes[s]
            self.scales[d] = self.scales[s]
            self.key_valid[d] = self.key_valid[s]

    def page(self, block, layer):
        return tuple(QuantizedKV(self.codes[block, layer, kv][None],
                                 self.scales[block, layer, kv][None, ..., None], torch.float32)
                     for kv in (0, 1))
