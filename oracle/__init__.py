"""CPU oracle for the INT8 paged-decode path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed CPU
baseline). The product package ``aster_amd`` never imports it: the HIP path
fails loudly when its extension is missing instead of falling back here.

Modules:
  reference_cpu  numpy restatement of sutiankang/aster's quantize_kv /
                 online_attention_statistics / merge_softmax and of the paged
                 runner's page-to-block assembly (each function cites the
                 reference file:line it follows).
  dense          independent brute-force fp64 dense softmax used to pin the
                 restatement (mirrors the reference test oracle).
"""
