"""Write the committed golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

Fixtures are data only: seeded inputs and the outputs of the pinned numpy oracle
(oracle/reference_cpu.py; see tests/test_oracle.py for what pins it).

  config1.npz        the config1 workload (tiny ragged INT8 paged decode): fp32
                     queries and K/V sources, block tables, context lengths, the
                     quantized arena (codes + scales) and the fp32 attention
                     output of the reference's page-by-page online softmax.
  quantize_seed76.npz  the reference's quantize_kv known-answer input
                     (tests/unit/test_hot_kv.py:22-42: torch.manual_seed(76),
                     randn(2,3,9,32), x[0,0,0]=0) with its codes and scales as
                     that test's independent numpy scalar formula defines them.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import reference_cpu as ref  # noqa: E402

DATA_SEED = 1001


def config1_inputs():
    """Seeded config-1 data: lengths {17,64,129,300}, 4q/4kv heads, D=64, bs=16,
    block tables = a permutation of a 64-block pool, fp32 N(0,1) q/K/V."""
    from aster_amd.workloads import config1

    w = config1()
    rng = np.random.default_rng(DATA_SEED)
    total = int(w.context_lens.sum())
    q = rng.standard_normal((w.num_seqs, w.num_q_heads, w.head_dim), dtype=np.float32)
    k = rng.standard_normal((total, w.num_kv_heads, w.head_dim), dtype=np.float32)
    v = rng.standard_normal((total, w.num_kv_heads, w.head_dim), dtype=np.float32)
    slots = np.concatenate([
        w.block_tables[r][np.arange(c) // 16].astype(np.int64) * 16 + np.arange(c) % 16
        for r, c in enumerate(w.context_lens.tolist())
    ])
    return w, q, k, v, slots


def config1_expected(w, q, k, v, slots):
    shape = (w.num_blocks, w.num_kv_heads, 16, w.head_dim)
    k_codes, v_codes = np.zeros(shape, np.int8), np.zeros(shape, np.int8)
    k_scales, v_scales = np.ones(shape[:3], np.float32), np.ones(shape[:3], np.float32)
    ref.quantize_append(k, v, slots, k_codes, k_scales, v_codes, v_scales, 16)
    out = ref.paged_attention(q, k_codes, k_scales, v_codes, v_scales, w.block_tables,
                              w.context_lens, block_size=16, scale=w.scale)
    return k_codes, k_scales, v_codes, v_scales, out


def seed76_input():
    import torch

    torch.manual_seed(76)
    x = torch.randn(2, 3, 9, 32)
    x[0, 0, 0] = 0
    return x.numpy()


def seed76_expected(x):
    """The reference test's independent scalar formula (test_hot_kv.py:29-34)."""
    scale = np.max(np.abs(x), axis=-1, keepdims=True) / 127.0
    scale = np.where(scale == 0, 1, scale).astype(np.float32)
    codes = np.rint(np.clip(x / scale, -127.0, 127.0)).astype(np.int8)
    return codes, scale


def main():
    w, q, k, v, slots = config1_inputs()
    k_codes, k_scales, v_codes, v_scales, out = config1_expected(w, q, k, v, slots)
    np.savez_compressed(
        os.path.join(HERE, "config1.npz"), q=q, k=k, v=v, slots=slots,
        block_tables=w.block_tables, context_lens=w.context_lens, k_codes=k_codes,
        k_scales=k_scales, v_codes=v_codes, v_scales=v_scales, out=out.astype(np.float32))
    x = seed76_input()
    codes, scale = seed76_expected(x)
    np.savez_compressed(os.path.join(HERE, "quantize_seed76.npz"), x=x, codes=codes, scales=scale)
    print("wrote config1.npz, quantize_seed76.npz")


if __name__ == "__main__":
    main()
