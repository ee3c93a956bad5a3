"""Explicit attention-backend contract of the HIP INT8 paged path.

Mirrors the reference's backend conventions (src/aster/optimization/fused_attention.py):
an explicitly selected backend name, an ``UnsupportedAttentionBackend`` (a
``ValueError``) raised for configurations the kernels do not cover -- never a
silent fallback (:59-62, :133-159) -- and a ``KernelWork`` record of what
actually ran (:64-73).
"""

from __future__ import annotations

from dataclasses import dataclass

BACKEND = "hip_int8_paged"


class UnsupportedAttentionBackend(ValueError):
    """The HIP backend has no kernel for this configuration; the caller must choose
    another backend explicitly (fused_attention.py:59-62)."""


@dataclass
class AttentionWork:
    """Tile counters (online_attention.py:18-26). For the HIP path a "key tile" is
    one 16-token cache block of one kv head read by the decode kernel."""

    query_tiles: int = 0
    key_tiles: int = 0
    max_score_elements: int = 0
    max_query_tile: int = 0
    max_key_tile: int = 0


@dataclass
class KernelWork(AttentionWork):
    """What actually executed (fused_attention.py:64-73). ``page_launches`` counts
    kernel launches (one per attention call plus the split-K merge when used)."""

    backend: str | None = None
    fallback_reason: str | None = None
    backward_tiles: int = 0
    max_backward_score_elements: int = 0
    saved_tensor_elements: int = 0
    page_launches: int = 0
    compiler_version: str | None = None
