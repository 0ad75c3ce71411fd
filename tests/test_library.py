"""The C-ABI library and the drop-in extension modules, without a GPU.

* libsanta_amd.so loads and exports every function include/santa_amd.h
  declares;
* the host-only entry points (planning, validation, error text) behave as
  the reference's host code (flash/santa_cuda.cpp:36-44,182-210;
  prop/santa_cuda.cpp:39-77,212-229);
* the extension modules import, expose the reference's names, argument
  order and defaults, and reject host tensors with the reference's message.

Compute entry points are only called with arguments that fail validation
before any HIP call.
"""
import ctypes
import os
import re
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "santa_amd.h")
LIB = os.path.join(REPO, "santa_amd", "libsanta_amd.so")

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE = 0, 1, 2, 3


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(santa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.skip("libsanta_amd.so not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB)
    L.santa_last_error.restype = ctypes.c_char_p
    L.santa_version.restype = ctypes.c_char_p
    return L


def test_header_symbols_exported(lib):
    names = declared_functions()
    assert len(names) >= 15, names
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (santa_[a-z0-9_]+)\b", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        assert hasattr(lib, n), n


def test_library_loads_in_a_fresh_process():
    code = f"import ctypes; L = ctypes.CDLL({LIB!r}); L.santa_version.restype = ctypes.c_char_p; print(L.santa_version().decode())"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "gfx950" in r.stdout


def _flash_plan(lib, L_storage, valid_len, block_n, S):
    out = [ctypes.c_int() for _ in range(4)]
    rc = lib.santa_flash_plan(ctypes.c_int64(L_storage), ctypes.c_int64(valid_len), ctypes.c_int64(block_n),
                              ctypes.c_int64(S), *[ctypes.byref(o) for o in out])
    return rc, [o.value for o in out]


def test_flash_plan_closed_forms(lib):
    assert _flash_plan(lib, 4096, -1, 0, 32) == (OK, [4096, 256, 16, 2])
    assert _flash_plan(lib, 32768, -1, 0, 256) == (OK, [32768, 256, 128, 2])
    assert _flash_plan(lib, 32832, -1, 0, 256) == (OK, [32832, 256, 129, 1])
    assert _flash_plan(lib, 131072, -1, 0, 512) == (OK, [131072, 256, 512, 1])
    assert _flash_plan(lib, 1536, -1, 0, 8) == (OK, [1536, 32, 48, 1])
    assert _flash_plan(lib, 3072, 2000, 0, 0) == (OK, [2000, 64, 32, 0])
    assert _flash_plan(lib, 100, -1, 64, 3) == (OK, [100, 64, 2, 1])


def test_flash_plan_errors(lib):
    rc, _ = _flash_plan(lib, 100, 101, 0, 8)
    assert rc == ERR_INVALID and b"valid_len exceeds storage length" in lib.santa_last_error()
    rc, _ = _flash_plan(lib, 100, -1, 128, 8)
    assert rc == ERR_INVALID and b"block_n must be 0 (auto) or one of {32,64,256}" in lib.santa_last_error()
    rc, _ = _flash_plan(lib, 100, -1, 0, 8)
    assert rc == OK and lib.santa_last_error() == b""


def _prop_plan(lib, L, H, KVH, D, block_n, env):
    out = [ctypes.c_int() for _ in range(3)]
    rc = lib.santa_prop_plan(L, H, KVH, D, ctypes.c_int64(block_n), env.encode() if env is not None else None,
                             *[ctypes.byref(o) for o in out])
    return rc, [o.value for o in out]


def test_prop_plan_modes(lib):
    # auto: vec when GH=4, D=128, block_n=256
    assert _prop_plan(lib, 5000, 32, 8, 128, 0, None) == (OK, [256, 20, 0])
    assert _prop_plan(lib, 1000, 32, 8, 128, 0, None) == (OK, [32, 32, 1])
    assert _prop_plan(lib, 5000, 64, 8, 128, 0, None) == (OK, [256, 20, 1])
    # SANTA_PASS1 is case-insensitive; "perhead" is the old name of "gqa"
    assert _prop_plan(lib, 5000, 32, 8, 128, 0, "GQA") == (OK, [256, 20, 1])
    assert _prop_plan(lib, 5000, 32, 8, 128, 0, "perhead") == (OK, [256, 20, 1])
    # vec forces block_n 256 when auto
    assert _prop_plan(lib, 1000, 32, 8, 128, 0, "vec") == (OK, [256, 4, 0])
    assert _prop_plan(lib, 1000, 32, 8, 128, 0, "gqa_vec") == (OK, [256, 4, 0])
    assert _prop_plan(lib, 1000, 32, 8, 128, 0, "bogus") == (OK, [32, 32, 1])
    rc, _ = _prop_plan(lib, 1000, 64, 8, 128, 0, "vec")
    assert rc == ERR_INVALID
    assert lib.santa_last_error() == b"SANTA_PASS1=vec requires GH=4, D=128, block_n=256. Got GH=8 D=128 block_n=256"
    rc, _ = _prop_plan(lib, 1000, 32, 8, 128, 40, None)
    assert rc == ERR_INVALID and b"Pass-1 WMMA-GQA requires D % 16 == 0 and block_n % 16 == 0" in lib.santa_last_error()


def test_compute_entry_points_validate_before_any_launch(lib):
    null = ctypes.c_void_p(0)
    # D = 64 is outside this build
    rc = lib.santa_flash_decode(null, null, null, 0, 1, 32, 8, 64, 100, 100, 32, 1, ctypes.c_uint64(1), null, null,
                                null, null, ctypes.c_size_t(0), null)
    assert rc == ERR_UNSUPPORTED and b"only D=128" in lib.santa_last_error()
    # GH = 2
    rc = lib.santa_flash_decode(null, null, null, 0, 1, 16, 8, 128, 100, 100, 32, 1, ctypes.c_uint64(1), null, null,
                                null, null, ctypes.c_size_t(0), null)
    assert rc == ERR_UNSUPPORTED and b"GH=2" in lib.santa_last_error()
    # valid_len > storage
    rc = lib.santa_flash_decode(null, null, null, 0, 1, 32, 8, 128, 200, 100, 32, 1, ctypes.c_uint64(1), null, null,
                                null, null, ctypes.c_size_t(0), null)
    assert rc == ERR_INVALID and b"valid_len exceeds storage length" in lib.santa_last_error()
    # bad dtype
    rc = lib.santa_flash_fused_tiles(null, null, null, 7, 1, 32, 8, 128, 100, 100, 32, 1, ctypes.c_uint64(1), null,
                                     null, null, null, null, null)
    assert rc == ERR_INVALID
    # prop: block_n, D and GH outside the build (any multiple of 16 up to 512,
    # a multiple of 16 up to 1024, at most 16)
    for bn in (100, 1024):
        rc = lib.santa_prop_decode(null, null, null, 0, 32, 8, 128, 1000, bn, 1, 8, ctypes.c_uint64(1), null, null,
                                   null, null, ctypes.c_size_t(0), null)
        assert rc == ERR_UNSUPPORTED and b"block_n a multiple of 16" in lib.santa_last_error()
    rc = lib.santa_prop_decode(null, null, null, 0, 32, 8, 40, 1000, 64, 1, 8, ctypes.c_uint64(1), null, null, null,
                               null, ctypes.c_size_t(0), null)
    assert rc == ERR_UNSUPPORTED and b"D a multiple of 16" in lib.santa_last_error()
    rc = lib.santa_prop_decode(null, null, null, 0, 32, 8, 1040, 1000, 64, 1, 8, ctypes.c_uint64(1), null, null, null,
                               null, ctypes.c_size_t(0), null)
    assert rc == ERR_UNSUPPORTED and b"up to 1024" in lib.santa_last_error()
    # D = 512 (above the reference-sized tuned kernels) passes validation
    rc = lib.santa_prop_decode(null, null, null, 0, 32, 8, 512, 1000, 64, 1, 8, ctypes.c_uint64(1), null, null, null,
                               null, ctypes.c_size_t(0), null)
    assert rc == ERR_INVALID and b"null pointer" in lib.santa_last_error()
    rc = lib.santa_prop_decode(null, null, null, 0, 64, 2, 128, 1000, 64, 1, 8, ctypes.c_uint64(1), null, null, null,
                               null, ctypes.c_size_t(0), null)
    assert rc == ERR_UNSUPPORTED and b"GH=32" in lib.santa_last_error()
    # prop: a generic shape passes validation and stops at the workspace
    rc = lib.santa_prop_decode(null, null, null, 0, 12, 4, 80, 1000, 48, 1, 8, ctypes.c_uint64(1), null, null, null,
                               null, ctypes.c_size_t(0), null)
    assert rc == ERR_INVALID and b"null pointer" in lib.santa_last_error()
    # prop: vec path with GH 8
    rc = lib.santa_prop_pass1(null, null, 0, 64, 8, 128, 1000, 256, 0, null, null, null, null)
    assert rc == ERR_INVALID and b"SANTA_PASS1=vec" in lib.santa_last_error()
    # budgets: empty shape
    rc = lib.santa_prop_tile_budgets(null, null, 0, 4, 8, ctypes.c_uint64(1), null, null, null, null, null)
    assert rc == ERR_INVALID


def test_linear_validates_before_any_launch(lib):
    """santa_rt_linear rejects what its staged rows cannot hold, and the
    runtime's shape predicate (which routes other shapes to F.linear) agrees
    on every rejected case; pointers are never dereferenced."""
    from santa_amd.runtime import _FusedOps

    p, null = ctypes.c_void_p(16), ctypes.c_void_p(0)
    assert lib.santa_rt_linear(null, p, p, 4, 64, 4096, 0, null) == ERR_INVALID
    assert lib.santa_rt_linear(ctypes.c_void_p(8), p, p, 4, 64, 4096, 0, null) == ERR_INVALID
    for M, K in [(0, 4096), (9, 4096), (4, 4100), (4, 16392), (8, 8200), (3, 20480), (1, 65544)]:
        assert lib.santa_rt_linear(p, p, p, M, 64, K, 0, null) == ERR_INVALID, (M, K)
        assert not _FusedOps.linear_fits(M, K), (M, K)
    assert b"linear" in lib.santa_last_error()
    for M, K in [(1, 65536), (2, 32768), (4, 16384), (4, 14336), (8, 8192), (3, 16384), (5, 8)]:
        assert _FusedOps.linear_fits(M, K), (M, K)
    # the RoPE form: odd D, pos outside the cache, null outputs, then the
    # product's own limits
    rope = lambda M, K, D, storage, pos, out=p: lib.santa_rt_linear_rope(p, p, M, K, p, p, out, p, p, 32, 8, D,
                                                                        ctypes.c_longlong(storage), pos, null)
    assert rope(4, 4096, 127, 100, 5) == ERR_INVALID
    assert rope(4, 4096, 128, 100, 100) == ERR_INVALID
    assert rope(4, 4096, 128, 100, -1) == ERR_INVALID
    assert rope(4, 4096, 128, 100, 5, null) == ERR_INVALID
    assert rope(9, 4096, 128, 100, 5) == ERR_INVALID
    assert rope(4, 16392, 128, 100, 5) == ERR_INVALID
    assert lib.santa_rt_argmax(null, 4, 100, p, null) == ERR_INVALID
    assert lib.santa_rt_argmax(p, 4, 0, p, null) == ERR_INVALID
    assert lib.santa_rt_argmax(p, -1, 100, p, null) == ERR_INVALID


def test_paged_entry_points_validate_the_page_table(lib):
    null = ctypes.c_void_p(0)
    table = (ctypes.c_int * 4)()  # host memory: only its address is checked before a launch

    def flash(page_size, num_pages, stride, max_len, block_table=table):
        return lib.santa_flash_decode_paged(null, null, null, 0, 1, 32, 8, 128, num_pages, page_size, block_table,
                                            stride, null, max_len, ctypes.c_longlong(1), 256, ctypes.c_int64(256),
                                            ctypes.c_uint64(1), null, null, null, null, ctypes.c_size_t(0), null)

    rc = flash(24, 4, 4, 64)
    assert rc == ERR_INVALID and b"page_size must be a power of two" in lib.santa_last_error()
    rc = flash(4, 4, 4, 16)
    assert rc == ERR_INVALID and b"page_size must be a power of two in [8" in lib.santa_last_error()
    rc = flash(16, 0, 4, 64)
    assert rc == ERR_INVALID and b"num_pages must be > 0" in lib.santa_last_error()
    rc = flash(16, 8, 3, 64)  # 64 tokens need 4 pages of 16
    assert rc == ERR_INVALID and b"block table too narrow" in lib.santa_last_error()
    rc = flash(16, 8, 4, 64, block_table=null)
    assert rc == ERR_INVALID and b"null pointer" in lib.santa_last_error()
    rc = lib.santa_prop_decode_paged(null, null, null, 0, 1, 32, 8, 128, 8, 12, table, 4, null, null, 64,
                                     ctypes.c_longlong(1), 256, 0, ctypes.c_uint64(1), null, null, null, null,
                                     ctypes.c_size_t(0), null)
    assert rc == ERR_INVALID and b"page_size must be a power of two" in lib.santa_last_error()


def test_workspace_sizes_are_host_only(lib):
    lib.santa_flash_workspace_size.restype = ctypes.c_size_t
    lib.santa_prop_workspace_size.restype = ctypes.c_size_t
    assert lib.santa_flash_workspace_size(8, 32, 8, 128, 128) > 0
    assert lib.santa_flash_workspace_size(8, 30, 8, 128, 128) == 0
    n = lib.santa_prop_workspace_size(32, 8, 128, 4096, 16)
    # stash [L, H] u16 alone is 256 KiB here
    assert n >= 4096 * 32 * 2 and n % 256 == 0


# ------------------------------------------------------------------ extension modules
def test_extension_surfaces():
    import torch

    import santa_flash_batch_cuda as flash
    import santa_prop_batch_cuda as prop

    # valid_len keeps the reference's int form and default; it is typed
    # `object` because the batched form also takes one length per sequence
    for fn in (flash.decode_systematic_scalar, flash.decode_systematic_batched):
        doc = fn.__doc__.splitlines()[0]
        assert re.search(r"\(q_h: .*, K_g: .*, V_g: .*, S: [\w.]*Int, seed: [\w.]*Int = 42, block_n: [\w.]*Int = 0, "
                         r"want_vrows: bool = False, valid_len: (?:[\w.]*Int|object) = -1\)", doc), doc
    doc = prop.decode_systematic_scalar.__doc__.splitlines()[0]
    assert re.search(r"\(q_h: .*, K_g: .*, V_g: .*, S: [\w.]*Int, seed: [\w.]*Int = 42, block_n: [\w.]*Int = 0, "
                     r"want_vrows: bool = False\)", doc), doc
    q = torch.zeros(32, 128, dtype=torch.bfloat16)
    K = torch.zeros(64, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="q_h must be CUDA"):
        flash.decode_systematic_scalar(q, K, K, 8)
    with pytest.raises(RuntimeError, match="q_h must be CUDA"):
        prop.decode_systematic_scalar(q, K, K, 8)
    with pytest.raises(TypeError):
        prop.decode_systematic_scalar(q, K, K, 8, valid_len=3)
    with pytest.raises(TypeError):
        flash.decode_systematic_scalar(q, K, K, 8, seed=-1)
    assert "gfx950" in flash._library_version() and "gfx950" in prop._library_version()


def test_noalloc_rejects_shapes_beyond_its_scratch(lib):
    """santa_flash_decode_noalloc checks the workspace its shape needs against
    its 16 MiB static scratch before any HIP call (so this runs without a
    GPU; the pointers are never dereferenced): B=1024, 64q/8kv, one 256-row
    tile each needs 8192 chunk partials of 8 heads, about 34 MB."""
    P, I, U64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64
    lib.santa_flash_decode_noalloc.argtypes = [P, P, P] + [I] * 9 + [U64, P, P, P, P]
    lib.santa_flash_workspace_size.restype = ctypes.c_size_t
    need = lib.santa_flash_workspace_size(1024, 64, 8, 128, 1)
    assert need > 16 << 20
    dummy = ctypes.c_void_p(0x1000)
    rc = lib.santa_flash_decode_noalloc(dummy, dummy, dummy, 0, 1024, 64, 8, 128, 256, 256, 256, 1, 1690, dummy, None,
                                        None, None)
    assert rc == ERR_WORKSPACE
    msg = lib.santa_last_error().decode()
    assert "needs" in msg and str(16 << 20) in msg and str(need) in msg, msg
    # argument errors come first, as in santa_flash_decode
    rc = lib.santa_flash_decode_noalloc(dummy, dummy, dummy, 0, 1, 32, 8, 64, 256, 256, 256, 1, 1690, dummy, None,
                                        None, None)
    assert rc == ERR_UNSUPPORTED and "D=128" in lib.santa_last_error().decode()
