"""ctypes binding of libmipaged.so, the C-ABI HIP library (declared in include/mipaged.h).

Loading is lazy and strict: any use of a kernel without the built library, or with
tensors that are not on a ROCm device, raises. There is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmipaged.so"

MIP_F32, MIP_F16, MIP_BF16 = 0, 1, 2
MIP_OK, MIP_E2BIG, MIP_EINVAL, MIP_EUNSUPPORTED = 0, -7, -22, -95
MIP_NOALLOC_SCRATCH_BYTES = 32 << 20
MIP_ALGO = {"auto": 0, "valu": 1, "mfma": 2, "stream": 3}

EXPORTED = (
    "mip_version",
    "mip_status_string",
    "mip_set_decode_algo",
    "mip_kv_append",
    "mip_rope_kv_append",
    "mip_paged_decode",
    "mip_paged_decode_append",
    "mip_paged_decode_append_noalloc",
    "mip_paged_decode_workspace",
    "mip_paged_decode_plan",
    "mip_paged_decode_plan_bytes",
    "mip_paged_prefill",
    "mip_copy_blocks",
    "mip_copy_blocks_host",
)

# Measurement helpers in the same library (include/mipaged_probe.h), outside the drop-in ABI.
PROBE_EXPORTED = ("mip_hbm_read_probe",)

_c = ctypes
_i32, _i64, _sz, _vp, _f32 = _c.c_int32, _c.c_int64, _c.c_size_t, _c.c_void_p, _c.c_float

_SIGNATURES = {
    "mip_version": (_c.c_int, []),
    "mip_status_string": (_c.c_char_p, [_c.c_int]),
    "mip_set_decode_algo": (_c.c_int, [_i32]),
    "mip_kv_append": (
        _c.c_int,
        [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "mip_rope_kv_append": (
        _c.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
         _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
    ),
    "mip_paged_decode": (
        _c.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp,
         _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp, _sz, _i32, _vp],
    ),
    "mip_paged_decode_append": (
        _c.c_int,
        [_vp, _vp, _i64, _i64, _i64, _i64, _vp,
         _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp,
         _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp, _sz, _i32, _vp],
    ),
    "mip_paged_decode_append_noalloc": (
        _c.c_int,
        [_vp, _vp, _i64, _i64, _i64, _i64, _vp,
         _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp,
         _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _i32, _vp],
    ),
    "mip_paged_decode_workspace": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "mip_paged_decode_plan_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "mip_paged_decode_plan": (
        _c.c_int,
        [_vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "mip_paged_prefill": (
        _c.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _vp],
    ),
    "mip_copy_blocks": (_c.c_int, [_vp, _vp, _vp, _i32, _i32, _i64, _i64, _vp]),
    "mip_copy_blocks_host": (_c.c_int, [_vp, _vp, _vp, _i32, _i32, _i64, _i64, _vp]),
    "mip_hbm_read_probe": (_c.c_int, [_vp, _i64, _vp, _i64, _i32, _vp, _i32, _i32, _vp]),
}

_lib: ctypes.CDLL | None = None


class NativeLibraryMissing(RuntimeError):
    pass


class NativeError(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library, with argument types set for every entry point."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise NativeLibraryMissing(
            f"{p} is not built; run `python mini-inference_amd/build.py` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def set_decode_algo(name: str) -> str:
    """Force the decode attention algorithm ("auto", "valu", "mfma", "stream"); returns the previous one.

    Process-wide (``mip_set_decode_algo``); meant for kernel comparisons and tests.
    """
    prev = load().mip_set_decode_algo(MIP_ALGO[name])
    if prev < 0:
        raise NativeError(f"mip_set_decode_algo({name!r}) failed: status {prev}")
    return next(k for k, v in MIP_ALGO.items() if v == prev)


def check(status: int, what: str) -> None:
    if status != MIP_OK:
        msg = load().mip_status_string(status).decode()
        raise NativeError(f"{what} failed: status {status} ({msg})")
