"""C-ABI library checks that need no GPU: it loads, exports every symbol the header
declares, sizes workspaces, and rejects bad arguments before touching a device."""

import ctypes
import os
import re

import pytest

from aster_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "aster_kv.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(astr_\w+)\s*\(", text,
                                 flags=re.M)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_native.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.astr_version().decode().endswith("gfx950")
    # the per-wave trace reader exists only in the separate trace build
    assert not hasattr(lib, "astr_trace_read")


def test_workspace_bytes():
    lib = _native.lib()
    ws = lib.astr_paged_attention_i8_workspace_bytes
    a = lambda x: (x + 255) // 256 * 256

    def partitioned(s, hq, d, parts):
        return a(s * hq * parts * d * 4) + a(s * hq * parts * 8)

    def streamk(s, hq, hkv, d, max_ctx, cus=256, packs=0, rows=0):
        # [block prefix over up to 512 work rows + 1, rows with blocks before each,
        # 4-int pack record per sequence][acc][(m, l)] of 2 slots per wave of slot
        # columns, then the packs' and packed sequences' own slots. Waves: at least
        # enough that a range of the cheapest blocks (pack blocks at no less than 16
        # against 50, plus 135 per work row) holds at most 1024 blocks.
        per_head = s * -(-max_ctx // 16)
        need = hkv * -(-(50 * per_head + 135 * (s + packs)) // (16 * 1024))
        cap = max(cus * 32, need)
        cap = -(-cap // 4) * 4
        g = hq // hkv
        cols = rows * g if packs else g
        slots = cap * 2 * cols + (2 * hkv * packs * rows * g if packs else 0)
        work_rows = 513
        return a((2 * (work_rows + 1) + 4 * s) * 4) + a(slots * d * 4) + a(slots * 2 * 4)

    # fixed partitions (S, Hq, Hkv, D, max_ctx, partition_tokens)
    assert ws(64, 32, 8, 128, 512, 512) == 0
    assert ws(64, 32, 8, 128, 4096, 512) == partitioned(64, 32, 128, 8)
    assert ws(16, 64, 8, 128, 32768, 512) == partitioned(16, 64, 128, 64)
    assert ws(4, 4, 4, 64, 300, 64) == partitioned(4, 4, 64, 5)
    assert ws(4, 4, 4, 64, 300, 100) == 0        # not a multiple of 64 -> invalid -> 0
    assert ws(4, 4, 4, 64, 9000, 8192) == 0      # partitions above 4096 tokens are invalid
    assert ws(4, 6, 4, 64, 300, 64) == 0         # q heads not a multiple of kv heads
    # automatic mode: room for stream-K (no GPU here: 256 CUs assumed) and the fallback
    assert ws(64, 32, 8, 128, 4096, 0) == max(streamk(64, 32, 8, 128, 4096),
                                              partitioned(64, 32, 128, 8))
    assert ws(16, 64, 8, 128, 32768, 0) == max(streamk(16, 64, 8, 128, 32768),
                                               partitioned(16, 64, 128, 64))
    # more than 512 sequences: partitioned only
    assert ws(600, 32, 8, 128, 4096, 0) == partitioned(600, 32, 128, 8)
    # prefix packs (S, Hq, Hkv, D, max_ctx, num_packs, rows_per_pack)
    shared = lib.astr_paged_attention_i8_shared_workspace_bytes
    assert shared(256, 32, 8, 128, 2560, 64, 4) == max(
        streamk(256, 32, 8, 128, 2560, packs=64, rows=4), partitioned(256, 32, 128, 5))
    assert shared(256, 32, 8, 128, 2560, 0, 0) == ws(256, 32, 8, 128, 2560, 0)
    assert shared(4, 8, 8, 256, 300, 2, 2) == max(
        streamk(4, 8, 8, 256, 300, packs=2, rows=2), partitioned(4, 8, 256, 1))
    assert shared(4, 8, 8, 64, 300, -1, 2) == 0 and shared(4, 8, 8, 64, 300, 1, 0) == 0


def _desc(**kw):
    base = dict(k_codes=16, v_codes=16, k_scales=16, v_scales=16, code_block_stride=2048,
                code_head_stride=2048, scale_block_stride=16, scale_head_stride=16,
                num_blocks=4, block_size=16, num_kv_heads=1, head_dim=128)
    base.update(kw)
    return _native.PagedKVDesc(**base)


def _attn(desc, **kw):
    args = dict(query=16, q_dtype=2, q_tok=128, q_head=128, out=16, o_tok=128, o_head=128,
                tables=16, bt_stride=4, lens=16, num_seqs=1, hq=1, max_ctx=64, scale=0.1,
                window=0, part=512, ws=None, ws_bytes=0, flag=16)
    args.update(kw)
    return _native.lib().astr_paged_attention_i8(
        ctypes.byref(desc) if desc is not None else None, *args.values(), None)


def test_attention_argument_errors_need_no_device():
    lib = _native.lib()
    assert _attn(None) == _native.ASTR_EINVAL
    assert "err_flag" in _native.last_error()
    assert _attn(_desc(), flag=None) == _native.ASTR_EINVAL
    assert _attn(_desc(block_size=8)) == _native.ASTR_EUNSUPPORTED
    assert _attn(_desc(num_kv_heads=2), hq=3) == _native.ASTR_EINVAL
    assert _attn(_desc(), scale=float("nan")) == _native.ASTR_EINVAL
    assert _attn(_desc(), scale=0.0) == _native.ASTR_EINVAL
    assert _attn(_desc(), window=-1) == _native.ASTR_EINVAL
    assert _attn(_desc(), max_ctx=65, bt_stride=4) == _native.ASTR_EINVAL
    assert _attn(_desc(), part=100) == _native.ASTR_EINVAL
    assert _attn(_desc(), q_dtype=7) == _native.ASTR_EUNSUPPORTED
    assert _attn(_desc(), query=17) == _native.ASTR_EINVAL  # misaligned rows
    assert _attn(_desc(head_dim=96, code_block_stride=1536, code_head_stride=1536),
                 q_tok=96, q_head=96, o_tok=96, o_head=96) == _native.ASTR_EUNSUPPORTED
    assert _attn(_desc(), max_ctx=1024, bt_stride=64, part=64) == _native.ASTR_EINVAL  # no workspace
    assert "workspace" in _native.last_error()
    assert _attn(_desc(), num_seqs=0) == 0  # empty batch: nothing to launch
    assert _attn(_desc(key_valid=20)) == _native.ASTR_EINVAL  # padding bytes misaligned
    assert "key_valid" in _native.last_error()
    del lib


def test_statistics_argument_errors_need_no_device():
    def stats_call(desc, stats=16, **kw):
        args = dict(query=16, q_tok=128, q_head=128, w=16, w_tok=128, w_head=128, stats=stats,
                    tables=16, bt_stride=4, lens=16, num_seqs=1, hq=1, max_ctx=64, scale=0.1,
                    window=0, part=512, ws=None, ws_bytes=0, flag=16)
        args.update(kw)
        return _native.lib().astr_paged_attention_i8_statistics(
            ctypes.byref(desc) if desc is not None else None, *args.values(), None)

    assert stats_call(_desc(), stats=None) == _native.ASTR_EINVAL
    assert "stats" in _native.last_error()
    assert stats_call(_desc(), stats=20) == _native.ASTR_EINVAL  # not 8-byte aligned
    assert stats_call(None) == _native.ASTR_EINVAL
    assert stats_call(_desc(), scale=0.0) == _native.ASTR_EINVAL
    assert stats_call(_desc(), q_tok=2) == _native.ASTR_EINVAL  # fp32 rows: 8 bytes apart
    assert stats_call(_desc(), num_seqs=0) == 0


def test_key_valid_argument_errors_need_no_device():
    f = _native.lib().astr_kv_write_key_valid
    flag = ctypes.c_int32(0)
    fp = ctypes.addressof(flag)
    assert f(None, 16, 16, 1, fp, None) == _native.ASTR_EINVAL
    assert f(ctypes.byref(_desc()), 16, 16, 1, fp, None) == _native.ASTR_EINVAL  # no key_valid
    assert "key_valid" in _native.last_error()
    d = _desc(key_valid=16)
    assert f(ctypes.byref(d), 16, 16, 1, None, None) == _native.ASTR_EINVAL
    assert f(ctypes.byref(d), 16, 16, -1, fp, None) == _native.ASTR_EINVAL
    assert f(ctypes.byref(d), None, 16, 1, fp, None) == _native.ASTR_EINVAL
    assert f(ctypes.byref(d), 16, 16, 0, fp, None) == 0  # no tokens: nothing to launch


def test_append_argument_errors_need_no_device():
    lib = _native.lib()
    f = lib.astr_kv_quantize_append_i8
    d = _desc()
    assert f(None, 16, 16, 0, 1, 128, 128, 128, 128, 16, 16, None) == _native.ASTR_EINVAL
    assert f(ctypes.byref(d), 16, 16, 0, -1, 128, 128, 128, 128, 16, 16, None) == _native.ASTR_EINVAL
    assert f(ctypes.byref(d), 16, 16, 0, 0, 128, 128, 128, 128, 16, 16, None) == 0  # no tokens
    assert f(ctypes.byref(d), 16, 16, 9, 1, 128, 128, 128, 128, 16, 16, None) == \
        _native.ASTR_EUNSUPPORTED
    big = _desc(head_dim=1024)
    assert f(ctypes.byref(big), 16, 16, 0, 1, 1024, 1024, 1024, 1024, 16, 16, None) == \
        _native.ASTR_EUNSUPPORTED
    assert f(ctypes.byref(d), None, 16, 0, 1, 128, 128, 128, 128, 16, 16, None) == _native.ASTR_EINVAL


def test_check_maps_codes_to_reference_exceptions():
    from aster_amd import UnsupportedAttentionBackend

    _attn(None)
    with pytest.raises(ValueError):
        _native.check(_native.ASTR_EINVAL, "x")
    with pytest.raises(UnsupportedAttentionBackend):
        _native.check(_native.ASTR_EUNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _native.check(98, "x")
    _native.check(0, "x")


def test_copy_blocks_rejects_bad_arguments_without_launching():
    lib = _native.lib()
    flag = ctypes.c_int32(0)
    buf = ctypes.create_string_buffer(256)
    p = ctypes.cast(buf, ctypes.c_void_p)
    fp = ctypes.addressof(flag)
    copy = lib.astr_kv_copy_blocks
    # nothing to move: success without touching the pointers
    assert copy(None, 16, None, 0, None, 16, None, 0, 16, 0, None, None) == 0
    assert copy(p, 16, None, 4, p, 16, None, 4, 0, 3, fp, None) == 0
    # negative sizes, missing pointers, block larger than its stride, identity beyond the end
    assert copy(p, 16, None, 4, p, 16, None, 4, 16, -1, fp, None) == _native.ASTR_EINVAL
    assert copy(None, 16, None, 4, p, 16, None, 4, 16, 1, fp, None) == _native.ASTR_EINVAL
    assert copy(p, 16, None, 4, p, 16, None, 4, 16, 1, None, None) == _native.ASTR_EINVAL
    assert copy(p, 8, None, 4, p, 16, None, 4, 16, 1, fp, None) == _native.ASTR_EINVAL
    assert copy(p, 16, None, 2, p, 16, None, 4, 16, 3, fp, None) == _native.ASTR_EINVAL
    assert copy(p, 16, None, 4, p, 16, None, 2, 16, 3, fp, None) == _native.ASTR_EINVAL
    assert "dst_blocks" in _native.last_error()


def test_prefix_pack_argument_errors_need_no_device():
    """astr_paged_attention_i8_shared checks its plan before any launch."""
    d = _desc(num_kv_heads=2)

    def shared(packs=16, num_packs=1, rows=2, window=0, hq=8):
        return _native.lib().astr_paged_attention_i8_shared(
            ctypes.byref(d), 16, 2, 128 * hq, 128, 16, 128 * hq, 128, 16, 4, 16, 1, hq, 64, 0.1,
            window, packs, num_packs, rows, None, 0, 16, None)

    assert shared(num_packs=-1) == _native.ASTR_EINVAL
    assert shared(packs=None) == _native.ASTR_EINVAL
    assert shared(packs=18) == _native.ASTR_EINVAL            # misaligned table
    assert shared(rows=1) == _native.ASTR_EINVAL
    assert shared(rows=5) == _native.ASTR_EINVAL              # 5 rows x G = 4 > 16 columns
    assert "rows_per_pack" in _native.last_error()
    assert shared(num_packs=129) == _native.ASTR_EUNSUPPORTED
    assert shared(num_packs=100, rows=4) == _native.ASTR_EUNSUPPORTED  # 400 pack rows > 256
    assert shared(window=8) == _native.ASTR_EUNSUPPORTED
    assert "window" in _native.last_error()


def test_merge_softmax_rejects_overlapping_outputs_without_launching():
    """Outputs that overlap an input or each other are refused before any launch: the
    threads of a row read both maxima while one of them writes the merged maximum."""
    f = _native.lib().astr_merge_softmax_f32
    rows, width = 4, 512
    row_b, wide_b = rows * 4, rows * width * 4
    base = 1 << 20  # fake device addresses: nothing is dereferenced on these paths
    lm, ll, ln = base, base + 4096, base + 8192
    rm, rl, rn = base + 16384, base + 20480, base + 65536
    om, ol, on = base + 131072, base + 135168, base + 139264
    assert wide_b <= 16384
    ins = (lm, ll, ln, rm, rl, rn)
    assert f(*ins, lm, ol, on, rows, width, None) == _native.ASTR_EINVAL  # max over left max
    assert "overlap" in _native.last_error()
    assert f(*ins, om, ol, rn, rows, width, None) == _native.ASTR_EINVAL  # numerator in place
    assert f(*ins, om, ol, ln + wide_b - 4, rows, width, None) == _native.ASTR_EINVAL  # partial
    assert f(*ins, om, om + row_b - 4, on, rows, width, None) == _native.ASTR_EINVAL  # out/out
    assert f(*ins, om, ol, on, 0, width, None) == 0  # no rows: nothing to launch


def test_planned_append_argument_errors_need_no_device():
    """astr_paged_attention_i8_planned_append checks its token rows before anything
    else: key/value/slot_mapping are required, bf16/fp16 only, rows 4-byte aligned and
    slots 8-byte aligned; a plan without sequences launches nothing."""
    from aster_amd.decode_plan import DecodePlanInfo

    info = DecodePlanInfo()
    info.num_seqs = 4

    def call(**kw):
        args = dict(query=16, q_dtype=2, q_tok=128, q_head=128, out=16, o_tok=128, o_head=128,
                    key=16, value=16, k_tok=1024, k_head=128, v_tok=1024, v_head=128,
                    slots=16, lens=16, hq=32, scale=0.1, plan=16, info=ctypes.byref(info),
                    ws=None, ws_bytes=0, flag=16)
        args.update(kw)
        return _native.lib().astr_paged_attention_i8_planned_append(
            ctypes.byref(_desc(num_kv_heads=8)), *args.values(), None)

    assert call(key=None) == _native.ASTR_EINVAL
    assert "key, value and slot_mapping" in _native.last_error()
    assert call(slots=None) == _native.ASTR_EINVAL
    assert call(q_dtype=0) == _native.ASTR_EUNSUPPORTED  # fp32 rows: appended separately
    assert call(key=18) == _native.ASTR_EINVAL            # rows not 4-byte aligned
    assert call(k_head=127) == _native.ASTR_EINVAL        # odd element stride
    assert call(slots=20) == _native.ASTR_EINVAL          # slots not 8-byte aligned
    assert "aligned" in _native.last_error()
    info.num_seqs = 0
    assert call(key=None) == 0                            # nothing to do
