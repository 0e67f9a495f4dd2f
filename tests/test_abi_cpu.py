"""CPU-side checks of the boundary: the library loads, exports every symbol
include/tqk.h declares, and its host-only functions validate descriptors.
No GPU work is launched."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib():
    from turboquant_pro_amd import _native as N
    if not os.path.exists(N.LIB_PATH):
        pytest.skip("libtqk.so not built (run __graft_entry__.build())")
    return N, N.lib()


def test_header_declares_exactly_the_bound_symbols():
    with open(os.path.join(ROOT, "include", "tqk.h")) as f:
        hdr = f.read()
    declared = set(re.findall(r"^(?:int|size_t)\s+(tqk_\w+)\(", hdr, re.M))
    from turboquant_pro_amd import _native as N
    assert declared == set(N.EXPORTS)


def test_library_exports_every_symbol():
    N, lib = _lib()
    for name in N.EXPORTS:
        assert hasattr(lib, name), name
    assert lib.tqk_version() == N.ABI_VERSION


def _desc(N, **kw):
    base = dict(n_kv_heads=8, n_q_heads=32, head_dim=128, hot_window=512, group_tokens=256,
                page_tokens=256, key_bits=4, value_bits=3, outliers_per_channel=5,
                outlier_cap=2560, max_pages_per_seq=126, max_groups_per_seq=126, hot_ring=512, n_pages=2016,
                sm_scale=1 / 128 ** 0.5)
    base.update(kw)
    return N.CacheDesc(**base)


def test_check_desc_status_codes():
    N, lib = _lib()
    ok = _desc(N)
    assert lib.tqk_check_desc(ctypes.byref(ok)) == N.TQK_OK
    # head dims the kernels are built for: 64, 128, 256
    for D, rc in ((64, N.TQK_OK), (256, N.TQK_OK), (96, N.TQK_EUNSUPPORTED), (512, N.TQK_EUNSUPPORTED)):
        assert lib.tqk_check_desc(ctypes.byref(_desc(N, head_dim=D))) == rc, D
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, value_bits=2))) == N.TQK_OK
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, value_bits=5))) == N.TQK_EUNSUPPORTED
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, zero_point=2))) == N.TQK_OK
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, zero_point=3))) == N.TQK_EINVAL
    # zero points belong to asym-NF4 keys
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, zero_point=1, key_grid=1))) == N.TQK_EINVAL
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, n_q_heads=12))) == N.TQK_EINVAL
    # any 1..8 query heads per kv head (Qwen2.5-7B: 28 over 4)
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, n_q_heads=56))) == N.TQK_OK
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, n_q_heads=72))) == N.TQK_EUNSUPPORTED
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, group_tokens=128))) == N.TQK_EINVAL
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, page_tokens=24))) == N.TQK_EINVAL
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, hot_window=1023, group_tokens=512))) == \
        N.TQK_EUNSUPPORTED
    assert lib.tqk_check_desc(ctypes.byref(_desc(N, n_pages=0))) == N.TQK_EINVAL
    assert lib.tqk_check_desc(None) == N.TQK_EINVAL


def test_workspace_bytes_cover_partials():
    """The workspace holds at least one (m, l, acc[D]) fp32 partial per query
    head per sequence and never shrinks as the context grows."""
    N, lib = _lib()
    d = _desc(N)
    a = lib.tqk_decode_workspace_bytes(ctypes.byref(d), 16, 8192)
    b = lib.tqk_decode_workspace_bytes(ctypes.byref(d), 16, 32768)
    assert 16 * d.n_q_heads * (d.head_dim + 2) * 4 <= a <= b
    assert lib.tqk_decode_workspace_bytes(ctypes.byref(d), 0, 10) == 0


def test_error_mapping():
    from turboquant_pro_amd import _native as N
    N.check(N.TQK_OK, "x")
    with pytest.raises(NotImplementedError):
        N.check(N.TQK_EUNSUPPORTED, "x")
    with pytest.raises(ValueError):
        N.check(N.TQK_EINVAL, "x")
    with pytest.raises(RuntimeError):
        N.check(N.TQK_EHIP, "x")


def _header_signatures():
    """{name: [param declarations]} for every entry point include/tqk.h declares."""
    with open(os.path.join(ROOT, "include", "tqk.h")) as f:
        hdr = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    sigs = {}
    for m in re.finditer(r"^(?:int|size_t)\s+(tqk_\w+)\(([^)]*)\);", hdr, re.M):
        params = [p.strip() for p in m.group(2).replace("\n", " ").split(",")]
        sigs[m.group(1)] = [] if params == ["void"] else params
    return sigs


def test_binding_declares_every_signature_with_64bit_pointers():
    """Every entry point gets argtypes matching the header's parameter count,
    and every pointer parameter is bound as c_void_p or a POINTER type: an
    undeclared ctypes call passes Python ints as 32-bit C ints, which
    truncates 64-bit device pointers (the cause of a GPU memory fault in a
    scratch harness that opened the library without this binding)."""
    N, lib = _lib()
    sigs = _header_signatures()
    assert set(sigs) == set(N.EXPORTS)
    for name, params in sigs.items():
        fn = getattr(lib, name)
        assert fn.argtypes is not None, f"{name}: argtypes not declared"
        assert len(fn.argtypes) == len(params), f"{name}: {len(fn.argtypes)} argtypes for {len(params)} params"
        for decl, ty in zip(params, fn.argtypes):
            if "*" in decl:
                ok = ty is ctypes.c_void_p or (isinstance(ty, type) and issubclass(ty, ctypes._Pointer))
                assert ok, f"{name}: pointer parameter '{decl}' bound as {ty}"
            elif "size_t" in decl:
                assert ty is ctypes.c_size_t, f"{name}: '{decl}' bound as {ty}"
            else:
                assert ty in (ctypes.c_int32, ctypes.c_int), f"{name}: '{decl}' bound as {ty}"
                assert "int32_t" in decl, f"{name}: '{decl}' is not a 32-bit integer"
        assert fn.restype in (ctypes.c_int, ctypes.c_size_t), f"{name}: restype {fn.restype}"


def test_noalloc_rejects_plans_beyond_its_scratch():
    """tqk_decode_noalloc returns TQK_EWORKSPACE for a step whose partials do
    not fit the 32 MiB scratch, before any GPU work (pointers are never
    dereferenced on this path)."""
    N, lib = _lib()
    d = _desc(N, n_pages=1 << 17, max_pages_per_seq=1 << 17, max_groups_per_seq=1 << 17)
    fake = ctypes.c_void_p(0x1000)
    ptrs = N.CachePtrs()
    rc = lib.tqk_decode_noalloc(ctypes.byref(d), ctypes.byref(ptrs), 1, fake, fake, 1 << 30, fake, None)
    assert rc == N.TQK_EWORKSPACE
    rc = lib.tqk_decode_noalloc(ctypes.byref(d), ctypes.byref(ptrs), 0, fake, fake, 100, fake, None)
    assert rc == N.TQK_EINVAL
