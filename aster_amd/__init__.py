"""aster_amd -- MI355X-native (gfx950) INT8 paged-KV decode hot path.

The path of sutiankang/aster that this package replaces: quantize-and-append of
new K/V tokens into an INT8 paged cache and ragged paged attention over it,
behind the reference's names (KVQuantization, QuantizedKV, quantize_kv,
KernelWork, UnsupportedAttentionBackend, PagedStatePool, PagedStateArchive,
PagedAttentionRunner) and a C-ABI library of hand-written HIP kernels
(include/aster_kv.h).
"""

from .attention_backend import BACKEND, AttentionWork, KernelWork, UnsupportedAttentionBackend
from .kv_quantization import KVQuantization, QuantizedKV, quantize_kv
from .offload import PagedStateArchive
from .online_attention import (AttentionBlock, SoftmaxState, merge_softmax, online_attention,
                               online_attention_statistics)
from .paged_kv import DEFAULT_PARTITION_TOKENS, PagedKVCache
from .paged_pool import (CacheCapacityError, KVStateCodec, PagedSequence, PagedStatePool, PageRef,
                         PageView, SlotReservation, StateError)
from .prefix_plan import PrefixPacks, plan_prefix_packs
from .runner import PagedAttentionRunner, PagedAttentionStep

__all__ = [
    "BACKEND", "AttentionWork", "KernelWork", "UnsupportedAttentionBackend",
    "KVQuantization", "QuantizedKV", "quantize_kv", "DEFAULT_PARTITION_TOKENS", "PagedKVCache",
    "KVStateCodec", "PagedStatePool", "PagedSequence", "PageRef", "PageView", "SlotReservation",
    "StateError", "CacheCapacityError", "PagedStateArchive", "PagedAttentionRunner",
    "PagedAttentionStep", "PrefixPacks", "plan_prefix_packs", "AttentionBlock", "SoftmaxState",
    "merge_softmax", "online_attention", "online_attention_statistics",
]
