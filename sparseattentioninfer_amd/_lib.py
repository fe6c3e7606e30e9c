"""ctypes binding of the C ABI in ``include/sparse_attn.h``.

The library is loaded once, from ``$SPARSE_ATTN_HIP_LIB`` or the in-tree
``_lib/libsparse_attn_hip.so``.  There is no fallback: a missing or
mismatched library raises :class:`HipLibraryError`.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

ABI_VERSION = 6
DTYPE_BF16 = 0
DTYPE_F16 = 1

_LIB = None
_LOCK = threading.Lock()

_i32, _i64, _f32, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_u64, _f64 = ctypes.c_uint64, ctypes.c_double

# Exported entry points and their argument types (mirrors include/sparse_attn.h).
SIGNATURES = {
    "sa_abi_version": (_i32, []),
    "sa_bigbird_block_mask": (_i32, [_vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _i32, _i32, _vp]),
    "sa_seeded_bigbird_block_mask": (_i32, [_vp, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _u64,
                                            _vp]),
    "sa_bernoulli_block_mask": (_i32, [_vp, _i64, _i64, _i32, _i32, _i32, _i32, _f64, _u64, _vp]),
    "sa_last_error": (ctypes.c_char_p, []),
    "sa_prefill": (_i32, [
        _i32,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64,
        _vp, _i64,
        _vp, _i64,
        _i32, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i32, _i32, _f32,
        _vp, _i64,
        _vp,
    ]),
    "sa_prefill_workspace_bytes": (_i64, []),
    "sa_block_mask_to_csr": (_i32, [
        _vp, _i64, _i64,
        _i32, _i32, _i32,
        _vp, _i64, _vp,
        _vp, _i64, _i64,
        _vp, _vp,
    ]),
    "sa_csr_to_tiles": (_i32, [
        _vp, _i64,
        _vp, _i64,
        _i32, _i32, _i32,
        _vp, _vp, _i64, _i64,
        _vp, _i64,
        _vp,
        _vp,
    ]),
    "sa_decode": (_i32, [
        _i32,
        _vp, _i64, _i64,
        _vp, _vp,
        _i64, _i64, _i64,
        _vp, _i64, _i32, _i32,
        _vp, _i32,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _i32,
        _vp, _i64, _i64,
        _i32, _i32, _i32, _i32, _i32, _f32,
        _i32, _vp, _i64,
        _vp,
    ]),
    "sa_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "sa_decode_noalloc": (_i32, [
        _i32,
        _vp, _i64, _i64,
        _vp, _vp,
        _i64, _i64, _i64,
        _vp, _i64, _i32, _i32,
        _vp, _i32,
        _vp, _i64, _i64,
        _vp, _i64, _i64,
        _i32,
        _vp, _i64, _i64,
        _i32, _i32, _i32, _i32, _i32, _f32,
        _i32, _vp,
    ]),
    "sa_decode_noalloc_scratch_bytes": (_i64, []),
    "sa_stream_read": (_i32, [_vp, _i64, _vp, _vp]),
    "sa_stream_read_workgroups": (_i32, []),
    "sa_mfma_rate": (_i32, [_i32, _i32, _vp, _i64, _vp]),
    "sa_lds_read_rate": (_i32, [_i32, _i32, _vp, _i64, _vp]),
    "sa_measure_cus": (_i32, []),
    "sa_stage_rate": (_i32, [_vp, _i64, _i32, _vp, _i64, _vp]),
    "sa_step_rate": (_i32, [_i32, _vp, _i64, _i32, _vp, _i64, _vp]),
    "sa_step_rate_threads": (_i32, [_i32]),
    "sa_prefill_timeline": (_i32, [
        _i32,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64, _i64, _i64,
        _vp, _i64,
        _vp, _i64,
        _i32, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i32, _i32, _f32,
        _vp, _i64,
        _vp, _i64,
        _vp,
    ]),
    "sa_prefill_timeline_words": (_i64, [_i32]),
    "sa_rmsnorm": (_i32, [_i32, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _f32, _vp]),
    "sa_qk_rope_kv": (_i32, [
        _i32, _vp, _i64, _vp, _vp, _vp, _vp,
        _vp, _i64, _i64,
        _vp, _vp, _i64, _i64, _i64,
        _vp, _i64, _i32, _i32,
        _i32, _i32, _i32, _i32, _i32, _f32, _vp,
    ]),
    "sa_swiglu": (_i32, [_i32, _vp, _i64, _vp, _i64, _i32, _i32, _vp]),
    "sa_gemm_skinny": (_i32, [_i32, _vp, _i64, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp]),
    "sa_gemm_skinny_swiglu": (_i32, [_i32, _vp, _i64, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp]),
}


class HipLibraryError(RuntimeError):
    """The HIP library is missing, unloadable or of another ABI version."""


class HipCallError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


def library_path() -> Path:
    env = os.environ.get("SPARSE_ATTN_HIP_LIB")
    if env:
        return Path(env)
    return Path(__file__).resolve().parent / "_lib" / "libsparse_attn_hip.so"


def load():
    """Returns the loaded ``ctypes.CDLL``; raises :class:`HipLibraryError` if unusable."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not path.exists():
            raise HipLibraryError(
                f"HIP library not found at {path}; build it with "
                "`python -m sparseattentioninfer_amd._build`")
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as e:
            raise HipLibraryError(f"cannot load {path}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise HipLibraryError(f"{path} does not export {name}")
            fn.restype = res
            fn.argtypes = args
        ver = lib.sa_abi_version()
        if ver != ABI_VERSION:
            raise HipLibraryError(f"{path} has ABI version {ver}, expected {ABI_VERSION}")
        _LIB = lib
        return lib


def check(fn: str, status: int) -> None:
    if status != 0:
        msg = load().sa_last_error().decode(errors="replace")
        raise HipCallError(fn, status, msg)
