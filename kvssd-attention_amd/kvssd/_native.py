"""ctypes binding of libkvssd_hip.so (the C ABI in include/kvssd_hip.h).

This replaces the reference's pybind/torch extension ``kvssd._C``
(csrc/bindings.cpp:16-45).  The library is loaded after ``import torch`` so the
dynamic loader resolves its ``libamdhip64.so.7`` dependency to the HIP runtime
torch already mapped: device pointers and streams from torch are then valid in
the library.  Loading fails loudly; nothing falls back to another path.
"""

from __future__ import annotations

import ctypes
import importlib.util
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the library load; see module docstring)

# The in-tree build; KVSSD_HIP_LIBRARY names another build of the same ABI
# (an instrumented one, say) for the whole process.
LIB_PATH = Path(os.environ.get("KVSSD_HIP_LIBRARY") or Path(__file__).resolve().parent / "libkvssd_hip.so").resolve()
LIB_PATH_OVERRIDDEN = bool(os.environ.get("KVSSD_HIP_LIBRARY"))
# the sources the in-tree build comes from (absent in an installed copy)
BUILD_SCRIPT = Path(__file__).resolve().parent.parent / "csrc" / "build.py"
ABI_VERSION = 5

DTYPE_F16, DTYPE_BF16, DTYPE_F32, DTYPE_F64 = 0, 1, 2, 3
KERNEL_AUTO, KERNEL_GENERAL, KERNEL_MFMA, KERNEL_STAGED = 0, 1, 2, 3
KERNEL_NAMES = {
    KERNEL_AUTO: "auto",
    KERNEL_GENERAL: "general",
    KERNEL_MFMA: "mfma",
    KERNEL_STAGED: "staged",
}

QUERY_DTYPES = {
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
    torch.float32: DTYPE_F32,
    torch.float64: DTYPE_F64,
}


class DecodeDesc(ctypes.Structure):
    _fields_ = [
        ("query_heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("block_tokens", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("query_dtype", ctypes.c_int32),
        ("num_selected", ctypes.c_int32),
        ("kernel", ctypes.c_int32),
        ("sm_scale", ctypes.c_double),
        ("out_query_dtype", ctypes.c_int32),  # 1: out in the query's dtype, 0: fp32
    ]


class RecordLayout(ctypes.Structure):
    """kvssd_record_layout (include/kvssd_hip.h)."""

    _fields_ = [(n, ctypes.c_int32) for n in ("bits", "block_tokens", "kv_heads", "head_dim", "group_size")]


# (name, restype, argtypes) for every entry point in include/kvssd_hip.h
_VP, _SZ, _I, _I64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int64
SIGNATURES = {
    "kvssd_hip_abi_version": (_I, []),
    "kvssd_hip_build_id": (ctypes.c_char_p, []),
    "kvssd_hip_device_ok": (_I, [_I, ctypes.c_char_p, _SZ]),
    "kvssd_hip_decode_workspace_bytes": (_I, [ctypes.POINTER(DecodeDesc), ctypes.POINTER(_SZ)]),
    "kvssd_hip_decode_kernel": (_I, [ctypes.POINTER(DecodeDesc), ctypes.POINTER(_I)]),
    "kvssd_hip_fused_decode": (_I, [ctypes.POINTER(DecodeDesc)] + [_VP] * 10 + [_SZ, _VP]),
    "kvssd_hip_fused_decode_static": (_I, [ctypes.POINTER(DecodeDesc)] + [_VP] * 10),
    "kvssd_hip_decode_partials": (_I, [ctypes.POINTER(DecodeDesc)] + [_VP] * 8 + [_SZ, _VP]),
    "kvssd_hip_decode_merge": (_I, [ctypes.POINTER(DecodeDesc), _VP, _SZ, _VP, _VP, _VP]),
    "kvssd_hip_merge_chunks": (_I, [_I, _I, _VP, _VP, _VP, _VP, _VP]),
    "kvssd_hip_unpack_codes": (_I, [_VP, _I, _I64, _VP, _VP]),
    "kvssd_hip_dequantize": (_I, [_VP, _VP, _I64, _I, _I, _I, _VP, _VP]),
    "kvssd_hip_record_bytes": (_I, [ctypes.POINTER(RecordLayout), ctypes.POINTER(_SZ)]),
    "kvssd_hip_gather_records": (_I, [ctypes.POINTER(RecordLayout), _VP, _SZ, _I, _I] + [_VP] * 7),
    "kvssd_hip_quantize": (_I, [_VP, _I, _I64, _I, _I, _I, _VP, _VP, _VP]),
    "kvssd_hip_encode_records": (_I, [ctypes.POINTER(RecordLayout), _I, _VP, _VP, _I64, _I, _I, _VP, _VP, _VP]),
    "kvssd_hip_vllm_sizes": (_I, [_I64, _I, _I, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "kvssd_hip_vllm_encode": (_I, [_VP, _I, _I64, _I, _I, _VP, _VP, _VP, _SZ, _VP]),
    "kvssd_hip_vllm_decode": (_I, [_VP, _I64, _I, _I, ctypes.c_uint32, _I, _VP, _VP, _VP, _SZ, _VP]),
    "kvssd_hip_memcpy_h2d_async": (_I, [_VP, _VP, _SZ, _VP]),
    "kvssd_hip_read_probe": (_I, [_VP, _SZ, _VP, _SZ, _VP]),
    "kvssd_hip_last_error": (ctypes.c_char_p, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


class NativeError(RuntimeError):
    """A runtime failure reported by libkvssd_hip (positive status)."""


_loaded_from: Path | None = None


def build_module():
    """csrc/build.py as a module (source hash, build), or None without sources."""
    if not BUILD_SCRIPT.exists():
        return None
    spec = importlib.util.spec_from_file_location("kvssd_hip_build", BUILD_SCRIPT)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def source_hash() -> str | None:
    """Hash of the HIP sources next to the package (what a fresh build's id would be)."""
    mod = build_module()
    return None if mod is None else mod.source_hash()


def load(path: str | Path | None = None) -> ctypes.CDLL:
    """Load and type the library once; raises RuntimeError when it is absent
    or stale, and when a different build is asked for after one was loaded.

    One process holds one build: two builds of the library carry the same
    translation-unit ids (``__hip_cuid_*``) for their device code, and a
    process that mapped two of them crashed at its first launches."""
    global _lib, _load_error, _loaded_from
    want = LIB_PATH if path is None else Path(path).resolve()
    with _lock:
        if _lib is not None:
            if want != _loaded_from:
                raise RuntimeError(
                    f"libkvssd_hip is already loaded from {_loaded_from}; one process holds one build "
                    f"(asked for {want}); run the other build in its own process"
                )
            return _lib
        if not want.exists():
            _load_error = f"{want.name} is not built; run python kvssd-attention_amd/csrc/build.py"
            raise RuntimeError(_load_error)
        try:
            lib = ctypes.CDLL(str(want))
        except OSError as exc:
            _load_error = f"cannot load {want}: {exc}"
            raise RuntimeError(_load_error) from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.kvssd_hip_abi_version()
        if version != ABI_VERSION:
            _load_error = f"{want.name} ABI {version} != expected {ABI_VERSION}; rebuild it"
            raise RuntimeError(_load_error)
        # the in-tree build must come from the sources beside it (a library
        # named by KVSSD_HIP_LIBRARY is the caller's own)
        if want == (Path(__file__).resolve().parent / "libkvssd_hip.so").resolve():
            have, tree = lib.kvssd_hip_build_id().decode(), source_hash()
            if tree is not None and have != tree:
                _load_error = (f"{want.name} was built from other sources (build {have}, tree {tree}); "
                               "rebuild it with python kvssd-attention_amd/csrc/build.py")
                raise RuntimeError(_load_error)
        _lib, _loaded_from = lib, want
        return lib


FASTCALL_SIGNATURE = "kvssd_hip_fused_decode/13"


def fused_decode_fast():
    """(call, entry) for calling the loaded library's kvssd_hip_fused_decode
    through the CPython module built beside it (csrc/fastcall.c):
    ``call(entry, desc, query, packed_k, packed_v, scales_k, scales_v,
    valid_tokens, block_table, out, lse, workspace, workspace_bytes, stream)``
    with every pointer an int (or None) and ``desc`` the address of a
    DecodeDesc, returning the status.  None when that module is absent, of
    another signature or, beside the in-tree library, from other sources than
    the library (callers then use the ctypes function)."""
    lib = load()
    try:
        from . import _fastcall
    except ImportError:
        return None
    if getattr(_fastcall, "SIGNATURE", None) != FASTCALL_SIGNATURE:
        return None
    if not LIB_PATH_OVERRIDDEN and getattr(_fastcall, "BUILD_ID", None) != lib.kvssd_hip_build_id().decode():
        return None
    return _fastcall.fused_decode, ctypes.cast(lib.kvssd_hip_fused_decode, ctypes.c_void_p).value


def build_id() -> str:
    """The loaded library's build id (a hash of the sources it came from)."""
    return load().kvssd_hip_build_id().decode()


def available() -> tuple[bool, str]:
    try:
        load()
        return True, "libkvssd_hip loaded"
    except RuntimeError as exc:
        return False, str(exc)


def last_error() -> str:
    msg = load().kvssd_hip_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Map a status to the reference's exception types (ValueError / RuntimeError)."""
    if rc == 0:
        return
    msg = last_error() or what
    if rc < 0:
        raise ValueError(msg)
    raise NativeError(f"{what} failed with hipError {rc}: {msg}")


def device_ok(index: int) -> tuple[bool, str]:
    buf = ctypes.create_string_buffer(256)
    ok = load().kvssd_hip_device_ok(index, buf, len(buf))
    return bool(ok), buf.value.decode()


def stream_handle(stream: torch.cuda.Stream | None) -> int:
    return 0 if stream is None else int(stream.cuda_stream)
