"""The C-ABI library loads and exports every entry point include/kvssd_hip.h
declares; argument errors surface without any GPU work."""

import ctypes
import re
from pathlib import Path

import pytest

from kvssd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "kvssd_hip.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(kvssd_hip_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(_native.SIGNATURES) == names
    assert lib.kvssd_hip_abi_version() == _native.ABI_VERSION


def test_build_id_matches_the_sources(tmp_path):
    # the in-tree library carries the hash of the sources it was built from,
    # both as an exported string and as a marked copy readable from the file
    mod = _native.build_module()
    assert mod is not None
    tree = mod.source_hash()
    assert _native.build_id() == tree == mod.built_id(_native.LIB_PATH)
    assert not mod.is_stale()
    # a library of other sources reads as stale (found without loading it)
    data = _native.LIB_PATH.read_bytes()
    other = tmp_path / "libother.so"
    other.write_bytes(data.replace(b"kvssd-build-id:" + tree.encode(), b"kvssd-build-id:" + b"0" * len(tree)))
    assert mod.built_id(other) == "0" * len(tree)
    assert mod.is_stale(other) and mod.is_stale(tmp_path / "absent.so")


def test_source_hash_covers_sources_header_and_flags(monkeypatch):
    mod = _native.build_module()
    base = mod.source_hash()
    monkeypatch.setattr(mod, "COMMON", mod.COMMON + ["-DSOMETHING"])
    assert mod.source_hash() != base
    monkeypatch.undo()
    header = mod.HEADER.read_bytes()
    real = Path.read_bytes
    monkeypatch.setattr(Path, "read_bytes", lambda p: real(p) + (b" " if p == mod.HEADER else b""))
    assert mod.source_hash() != base
    monkeypatch.undo()
    assert mod.source_hash() == base and mod.HEADER.read_bytes() == header


def test_argument_errors_are_negative_with_messages():
    lib = _native.load()
    desc = _native.DecodeDesc(32, 8, 128, 4, 128, 3, 32, 0, 0, 0, 0.1)
    n = ctypes.c_size_t(0)
    rc = lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n))
    assert rc < 0 and "bits must be 2 or 4" in _native.last_error()
    with pytest.raises(ValueError, match="bits"):
        _native.check(rc, "workspace")
    desc.bits, desc.query_heads = 4, 30
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) < 0
    assert "divisible" in _native.last_error()
    desc.query_heads, desc.head_dim = 32, 512
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) < 0
    desc.head_dim, desc.group_size = 128, 48
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) < 0
    assert "group_size" in _native.last_error()
    desc.group_size = 32
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0 and n.value > 0
    assert lib.kvssd_hip_unpack_codes(None, 3, 4, None, None) < 0
    assert lib.kvssd_hip_read_probe(None, 17, None, 8192, None) < 0 and "multiple of 16" in _native.last_error()
    assert lib.kvssd_hip_read_probe(16, 32, 16, 100, None) < 0 and "8192" in _native.last_error()
    assert lib.kvssd_hip_read_probe(8, 32, 16, 8192, None) < 0 and "aligned" in _native.last_error()
    assert lib.kvssd_hip_merge_chunks(0, 8, None, None, None, None, None) < 0


def test_descriptor_layout_and_output_dtype_flag():
    # the C struct: ten int32, a double at byte 40, then out_query_dtype at 48
    # (padded to 56); a zeroed field keeps the fp32 output of earlier callers
    assert ctypes.sizeof(_native.DecodeDesc) == 56
    assert _native.DecodeDesc.sm_scale.offset == 40 and _native.DecodeDesc.out_query_dtype.offset == 48
    lib = _native.load()
    desc = _native.DecodeDesc(32, 8, 128, 4, 128, 4, 32, 0, 0, 0, 0.1)
    assert desc.out_query_dtype == 0
    n = ctypes.c_size_t(0)
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0
    fp32_bytes = n.value
    desc.out_query_dtype = 1
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0
    assert n.value == fp32_bytes  # the partials do not depend on the output dtype
    desc.out_query_dtype = 2
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) < 0
    assert "out_query_dtype" in _native.last_error()


def test_kernel_choice_is_reported():
    lib = _native.load()
    k = ctypes.c_int(-1)
    desc = _native.DecodeDesc(4, 2, 32, 2, 8, 4, 16, 2, 0, 0, 0.1)
    assert lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(k)) == 0
    assert k.value == _native.KERNEL_GENERAL
    desc.kernel = _native.KERNEL_GENERAL
    assert lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(k)) == 0


def test_record_codec_sizes_and_argument_errors():
    # sizes and argument checks of the record and vLLM codecs need no GPU
    lib = _native.load()
    n = ctypes.c_size_t(0)
    lay = _native.RecordLayout(4, 128, 8, 128, 32)
    assert lib.kvssd_hip_record_bytes(ctypes.byref(lay), ctypes.byref(n)) == 0 and n.value == 151552
    lay2 = _native.RecordLayout(2, 128, 8, 128, 32)
    assert lib.kvssd_hip_record_bytes(ctypes.byref(lay2), ctypes.byref(n)) == 0 and n.value == 86016
    bad = _native.RecordLayout(3, 128, 8, 128, 32)
    assert lib.kvssd_hip_record_bytes(ctypes.byref(bad), ctypes.byref(n)) < 0
    assert "bits" in _native.last_error()
    st = (ctypes.c_int32 * 1)()
    assert lib.kvssd_hip_gather_records(ctypes.byref(lay), None, 151552, 1, 1, *([None] * 6), st, None) < 0
    assert lib.kvssd_hip_gather_records(ctypes.byref(lay), 4, 100, 1, 1, *([8] * 6), st, None) < 0  # stride too small
    assert lib.kvssd_hip_quantize(None, 0, 4, 100, 4, 32, None, None, None) < 0  # 100 % 32
    rec, scratch = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.kvssd_hip_vllm_sizes(8388608, 4, 32, ctypes.byref(rec), ctypes.byref(scratch)) == 0
    assert rec.value == 4722688 and scratch.value == 288 * 4 + 4  # 4,718,592-byte payload: 288 rows
    assert lib.kvssd_hip_vllm_sizes(40, 4, 32, ctypes.byref(rec), ctypes.byref(scratch)) < 0
    assert "not divisible by group_size=32" in _native.last_error()
    assert lib.kvssd_hip_vllm_sizes(1 << 27, 4, 32, ctypes.byref(rec), ctypes.byref(scratch)) < 0  # > 16 MiB payload
    assert lib.kvssd_hip_vllm_encode(None, 3, 64, 4, 32, None, None, None, 0, None) < 0  # float64
    assert lib.kvssd_hip_vllm_decode(None, 64, 4, 32, 0, 0, None, None, None, 0, None) < 0


def _need(msg: str) -> int:
    m = re.search(r"need (\d+) bytes", msg)
    assert m, msg
    return int(m.group(1))


@pytest.mark.parametrize("selected", [1, 33, 700])
def test_num_selected_plans_the_same_splits_in_every_phase(selected):
    # a table of `selected` ids out of 2048 blocks: the workspace query, the
    # partials phase (table given) and the merge phase (no table pointer) agree
    # on the split plan; none of these calls reaches a launch
    lib = _native.load()
    desc = _native.DecodeDesc(64, 8, 128, 2048, 128, 4, 32, 0, selected, 0, 0.1)
    n = ctypes.c_size_t(0)
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0
    fake_table = ctypes.c_void_p(256)
    rc = lib.kvssd_hip_decode_partials(ctypes.byref(desc), *([None] * 6), fake_table, None, 0, None)
    assert rc < 0
    need_partials = _need(_native.last_error())
    rc = lib.kvssd_hip_decode_merge(ctypes.byref(desc), None, 0, None, None, None)
    assert rc < 0
    need_merge = _need(_native.last_error())
    assert n.value == need_partials == need_merge
    # the same count as a compacted batch of `selected` blocks plans alike
    compact = _native.DecodeDesc(64, 8, 128, selected, 128, 4, 32, 0, 0, 0, 0.1)
    m = ctypes.c_size_t(0)
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(compact), ctypes.byref(m)) == 0
    assert m.value == n.value


def test_num_selected_without_a_table_is_an_argument_error():
    lib = _native.load()
    desc = _native.DecodeDesc(32, 8, 128, 64, 128, 4, 32, 0, 5, 0, 0.1)
    fake = [ctypes.c_void_p(256)] * 6
    work = ctypes.c_void_p(256)
    rc = lib.kvssd_hip_decode_partials(ctypes.byref(desc), *fake, None, work, 1 << 30, None)
    assert rc < 0 and "num_selected must be 0 when block_table is NULL" in _native.last_error()
    rc = lib.kvssd_hip_fused_decode(ctypes.byref(desc), *fake, None, ctypes.c_void_p(256), ctypes.c_void_p(256),
                                    work, 1 << 30, None)
    assert rc < 0 and "num_selected must be 0" in _native.last_error()
    desc.num_selected = -1
    n = ctypes.c_size_t(0)
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) < 0
    assert "num_selected must be >= 0" in _native.last_error()
    # a table with no entries
    desc.num_selected = 0
    rc = lib.kvssd_hip_decode_partials(ctypes.byref(desc), *fake, ctypes.c_void_p(256), work, 1 << 30, None)
    assert rc < 0 and "at least one block is required" in _native.last_error()


def test_a_second_build_is_refused_in_the_same_process(tmp_path):
    lib = _native.load()
    assert _native.load(_native.LIB_PATH) is lib
    other = tmp_path / "libkvssd_hip_other.so"
    other.write_bytes(_native.LIB_PATH.read_bytes())
    with pytest.raises(RuntimeError, match="one process holds one build"):
        _native.load(other)
    assert _native.load() is lib


def test_static_scratch_decode_rejects_shapes_beyond_its_limit():
    # 64 query heads over one kv head, head_dim 256, 4096 blocks: 1024 splits of
    # 64 x 258 floats = 67 MB of partials, more than the 16 MiB scratch; the
    # call fails before any device work
    lib = _native.load()
    desc = _native.DecodeDesc(64, 1, 256, 4096, 16, 4, 32, 2, 0, 0, 0.1)
    n = ctypes.c_size_t(0)
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0 and n.value > 16 << 20
    fake = [ctypes.c_void_p(256)] * 6
    rc = lib.kvssd_hip_fused_decode_static(ctypes.byref(desc), *fake, None, ctypes.c_void_p(256), ctypes.c_void_p(256),
                                           None)
    assert rc < 0 and "static scratch" in _native.last_error()
    assert lib.kvssd_hip_fused_decode_static(ctypes.byref(desc), *fake, None, None, None, None) < 0


def test_auto_takes_the_matrix_core_kernel_for_small_decodes():
    # at most 512 (kv head, attended block) pairs: the one-wave matrix-core
    # kernel under AUTO (it spreads them over every CU); the staged kernel
    # beyond, and whenever it is asked for
    lib = _native.load()
    k = ctypes.c_int(-1)

    def choice(num_blocks, num_selected=0, kernel=_native.KERNEL_AUTO):
        desc = _native.DecodeDesc(32, 8, 128, num_blocks, 128, 4, 32, 0, num_selected, kernel, 0.1)
        assert lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(k)) == 0
        return k.value

    assert choice(32) == _native.KERNEL_MFMA  # 4K tokens: 256 pairs
    assert choice(64) == _native.KERNEL_MFMA  # 512 pairs
    assert choice(65) == _native.KERNEL_STAGED
    assert choice(1024) == _native.KERNEL_STAGED
    assert choice(2048, num_selected=33) == _native.KERNEL_MFMA  # a 33-block selection of a long context
    assert choice(32, kernel=_native.KERNEL_STAGED) == _native.KERNEL_STAGED
    # 8 query heads per kv head, any query dtype: small decodes give each query
    # quad a workgroup of its own, so the two-quad form (which spills with a
    # two-part fp32 query) is not involved and the matrix-core kernel is taken
    for dtype in (_native.DTYPE_F32, _native.DTYPE_F16, _native.DTYPE_F64):
        desc = _native.DecodeDesc(64, 8, 128, 32, 128, 4, 32, dtype, 0, 0, 0.1)
        assert lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(k)) == 0 and k.value == _native.KERNEL_MFMA
        desc.num_blocks = 65
        assert lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(k)) == 0 and k.value == _native.KERNEL_STAGED


def test_fast_call_module_matches_the_ctypes_call():
    # the CPython module built with the library calls the same entry point
    # with the same argument positions: each vector below fails a different
    # argument check (and at least two, so no mapping could reach a launch),
    # and both routes report the same status and message
    fast = _native.fused_decode_fast()
    assert fast is not None, "the CPython fast-call module was not built beside the library"
    call, entry = fast
    lib = _native.load()
    assert entry == ctypes.cast(lib.kvssd_hip_fused_decode, ctypes.c_void_p).value
    fake = 256

    def both(desc, query, table, out, lse, work, nbytes):
        ptrs = [query, fake, fake, fake, fake, fake, table, out, lse, work]
        rc_c = lib.kvssd_hip_fused_decode(ctypes.byref(desc), *ptrs[:9], ptrs[9], nbytes, None)
        msg_c = _native.last_error()
        rc_f = call(entry, ctypes.addressof(desc), *ptrs, nbytes, None)
        msg_f = _native.last_error()
        assert rc_c < 0 and (rc_f, msg_f) == (rc_c, msg_c)
        return msg_f

    desc = _native.DecodeDesc(32, 8, 128, 64, 128, 4, 32, 0, 0, 0, 0.1)
    assert "a required buffer pointer is NULL" in both(desc, fake, None, None, fake, fake, 1)  # out
    assert "a required buffer pointer is NULL" in both(desc, fake, None, fake, None, fake, 1)  # lse
    need = _need(both(desc, None, None, fake, fake, fake, 1))  # workspace bytes
    assert need > 1
    assert "workspace too small" in both(desc, None, None, fake, fake, None, 1 << 30)  # workspace pointer
    desc.num_selected = 5
    assert "num_selected must be 0 when block_table is NULL" in both(desc, fake, None, fake, fake, fake, 1)
    desc.num_selected = 0
    assert "at least one block is required" in both(desc, None, fake, fake, fake, fake, 1)  # table
    with pytest.raises(TypeError, match="14 arguments"):
        call(entry, ctypes.addressof(desc))


def test_fast_call_module_carries_the_build_id(monkeypatch):
    # built from the same sources as the library (the id is also in the file,
    # where the build script reads it), and refused when it is not
    from kvssd import _fastcall

    mod = _native.build_module()
    tree = mod.source_hash()
    assert _fastcall.BUILD_ID == _native.build_id() == tree == mod.built_id(mod.FASTCALL_OUT)
    assert _native.fused_decode_fast() is not None
    monkeypatch.setattr(_fastcall, "BUILD_ID", "0" * len(tree))
    assert _native.fused_decode_fast() is None
    monkeypatch.undo()
    monkeypatch.setattr(_fastcall, "SIGNATURE", "kvssd_hip_fused_decode/12")
    assert _native.fused_decode_fast() is None
