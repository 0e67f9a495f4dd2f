"""ctypes binding of the C ABI in ``include/tqk.h`` (``lib/libtqk.so``).

The library is the only compute path: there is no CPU fallback.  Loading
fails loudly when the library has not been built, and every call maps the
returned status to the Python exception the reference raises for the same
condition (TQK_EUNSUPPORTED -> NotImplementedError, TQK_EINVAL -> ValueError).
"""

from __future__ import annotations

import ctypes
import os

from ._build import LIB_PATH

TQK_OK = 0
TQK_EINVAL = 1
TQK_EUNSUPPORTED = 2
TQK_EHIP = 3
TQK_EWORKSPACE = 4

ABI_VERSION = 9

# Every symbol include/tqk.h declares (checked by the CPU test suite).
EXPORTS = (
    "tqk_version", "tqk_check_desc", "tqk_decode_workspace_bytes", "tqk_decode",
    "tqk_decode_noalloc", "tqk_decode_partials", "tqk_decode_splits", "tqk_decode_merge", "tqk_encode_groups",
    "tqk_append_hot", "tqk_dequant_groups", "tqk_encode_key_block", "tqk_encode_value_block",
    "tqk_dequant_key_block", "tqk_dequant_value_block",
)


class CacheDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "n_kv_heads", "n_q_heads", "head_dim", "hot_window", "group_tokens", "page_tokens",
        "key_bits", "value_bits", "outliers_per_channel", "outlier_cap",
        "max_pages_per_seq", "max_groups_per_seq", "hot_ring", "n_pages")] + [
        ("sm_scale", ctypes.c_float), ("key_grid", ctypes.c_int32), ("zero_point", ctypes.c_int32),
        ("input_f32", ctypes.c_int32), ("dc_mask", ctypes.c_uint32 * 8)]


class CachePtrs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "kcodes", "vcodes", "vnorm", "gscale", "gmean", "ocount", "oent", "hot_k", "hot_v",
        "block_table", "group_table", "pi", "pi_t", "vcent", "vbnd", "zp_mean", "knorm")]


class BlockDesc(ctypes.Structure):
    """``tqk_block_desc``: one (B, H, S, D) block for the stateless quantizers."""
    _fields_ = [(n, ctypes.c_int32) for n in (
        "batch", "n_heads", "tokens", "head_dim", "bits", "key_grid", "zero_point",
        "outliers_per_channel", "outlier_cap", "input_f32")] + [("dc_mask", ctypes.c_uint32 * 8)]


_lib = None


def load(path: str) -> ctypes.CDLL:
    """Open a build of the library at ``path`` with every entry point's C
    signature declared (pointer arguments stay 64-bit) and its ABI checked."""
    l_ = ctypes.CDLL(path)
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t
    pd, pp, pb = ctypes.POINTER(CacheDesc), ctypes.POINTER(CachePtrs), ctypes.POINTER(BlockDesc)
    sig = {
        "tqk_version": ([], ctypes.c_int),
        "tqk_check_desc": ([pd], ctypes.c_int),
        "tqk_decode_workspace_bytes": ([pd, i32, i32], sz),
        "tqk_decode": ([pd, pp, i32, vp, vp, i32, vp, vp, sz, vp], ctypes.c_int),
        "tqk_decode_noalloc": ([pd, pp, i32, vp, vp, i32, vp, vp], ctypes.c_int),
        "tqk_decode_partials": ([pd, pp, i32, vp, vp, i32, vp, vp, vp, vp, sz, vp], ctypes.c_int),
        "tqk_decode_splits": ([pd, pp, i32, vp, vp, i32, vp, sz, vp], ctypes.c_int),
        "tqk_decode_merge": ([pd, pp, i32, i32, vp, vp, sz, vp], ctypes.c_int),
        "tqk_encode_groups": ([pd, pp, i32, i32, vp, vp, vp, vp, i32, vp, vp], ctypes.c_int),
        "tqk_append_hot": ([pd, pp, i32, vp, vp, vp, vp, vp, i32, vp], ctypes.c_int),
        "tqk_dequant_groups": ([pd, pp, i32, vp, vp, vp, vp], ctypes.c_int),
        "tqk_encode_key_block": ([pb, vp, vp, vp, vp, vp, vp, vp, vp, vp], ctypes.c_int),
        "tqk_encode_value_block": ([pb, vp, vp, vp, vp, vp, vp], ctypes.c_int),
        "tqk_dequant_key_block": ([pb, vp, vp, vp, i32, vp, vp, vp, vp], ctypes.c_int),
        "tqk_dequant_value_block": ([pb, vp, vp, vp, vp, vp, vp], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(l_, name)
        fn.argtypes = args
        fn.restype = res
    if l_.tqk_version() != ABI_VERSION:
        raise RuntimeError(f"libtqk ABI {l_.tqk_version()} != expected {ABI_VERSION}")
    return l_


def lib() -> ctypes.CDLL:
    """The loaded library (built in-tree by ``__graft_entry__.build()``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the gfx950 library first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        _lib = load(LIB_PATH)
    return _lib


def check(rc: int, what: str) -> None:
    """Map a TQK status to the exception the reference path raises."""
    if rc == TQK_OK:
        return
    if rc == TQK_EUNSUPPORTED:
        raise NotImplementedError(f"{what}: configuration has no gfx950 form")
    if rc == TQK_EINVAL:
        raise ValueError(f"{what}: invalid argument")
    if rc == TQK_EWORKSPACE:
        raise ValueError(f"{what}: workspace too small")
    raise RuntimeError(f"{what}: HIP error (status {rc})")
