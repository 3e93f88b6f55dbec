"""The drop-in boundary, checked without a GPU.

* libflock_attn.so loads and exports every function include/*.h declares,
  and the ctypes table in flock_amd/_lib.py binds exactly that set.
* Host-side guards run before any launch and return the documented status
  (the reference throws from Layer before encoding: layer.ts:575, 689-698;
  lib.ts:504-506). Garbage non-null pointers are safe here because a rejected
  call never dereferences them.
"""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from flock_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("flock_attn.h", "flock_q8.h",
                                                      "flock_wire.h", "flock_graph.h")]
FAKE = 0x1000  # never dereferenced: every call below fails validation first


def declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(flk_\w+)\s*\(", text))
    return names


def test_every_header_is_listed():
    assert sorted(os.path.basename(h) for h in HEADERS) == sorted(
        f for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h"))


def declared_arity() -> dict[str, int]:
    """Entry point -> parameter count of its prototype in include/*.h."""
    out = {}
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for name, params in re.findall(r"\b(flk_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            params = params.strip()
            out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_header_and_binding_agree():
    assert declared_functions() == set(_lib.SIGNATURES)
    arity = declared_arity()
    assert set(arity) == declared_functions()
    for name, (_, args) in _lib.SIGNATURES.items():
        assert len(args) == arity[name], (name, len(args), arity[name])


def deno_binding() -> dict[str, int]:
    """Entry point -> parameter count of the Deno.dlopen table in
    flock_amd/deno/hip_attn.ts (the TypeScript host's binding)."""
    text = open(os.path.join(ROOT, "flock_amd", "deno", "hip_attn.ts")).read()
    table = {}
    for name, params in re.findall(r"\b(flk_\w+):\s*\{\s*parameters:\s*\[(.*?)\]", text, flags=re.S):
        table[name] = len([p for p in params.split(",") if p.strip()])
    return table


def test_deno_binding_lists_every_declared_symbol_with_its_arity():
    """The Deno binding binds every entry point, no more, each with as many
    parameters as its C prototype (and the ctypes table) has."""
    table = deno_binding()
    assert set(table) == declared_functions(), (declared_functions() - set(table),
                                                set(table) - declared_functions())
    for name, n in table.items():
        assert n == len(_lib.SIGNATURES[name][1]), (name, n, len(_lib.SIGNATURES[name][1]))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    out = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    exported = set(re.findall(r"\b(flk_\w+)$", out, flags=re.M))
    assert declared_functions() <= exported


def test_version_and_empty_error():
    L = _lib.lib()
    assert b"gfx950" in L.flk_version()


def code_and_msg(rc):
    return rc, _lib.lib().flk_last_error().decode()


def test_decode_layer_cache_full_is_rejected_before_launch():
    L = _lib.lib()
    rc, msg = code_and_msg(L.flk_decode_layer(*([FAKE] * 6), 1e-6, 0, *([FAKE] * 4),
                                              2048, 16, 8, 128, 2048, FAKE, 1 << 30))
    assert rc == _lib.FLK_ERR_CACHE_FULL and "2048" in msg


def test_prologue_cache_overflow_is_rejected():
    L = _lib.lib()
    rc, msg = code_and_msg(L.flk_qk_prologue(*([FAKE] * 6), 1e-6, 0, *([FAKE] * 3),
                                             5, 2046, 16, 8, 128, 2048))
    assert rc == _lib.FLK_ERR_CACHE_FULL and "2046 + 5" in msg


@pytest.mark.parametrize("H,Hkv,d,code", [(16, 8, 96, _lib.FLK_ERR_UNSUPPORTED),
                                          (16, 6, 128, _lib.FLK_ERR_ARG),
                                          (32, 2, 128, _lib.FLK_ERR_UNSUPPORTED),
                                          (0, 8, 128, _lib.FLK_ERR_ARG)])
def test_unsupported_shapes(H, Hkv, d, code):
    L = _lib.lib()
    rc = L.flk_attn_decode(FAKE, FAKE, FAKE, FAKE, H, Hkv, d, 10, FAKE, 1 << 30)
    assert rc == code


def test_null_pointer_and_zero_sizes():
    L = _lib.lib()
    assert L.flk_attn_decode(None, FAKE, FAKE, FAKE, 16, 8, 128, 10, FAKE, 1 << 30) == _lib.FLK_ERR_ARG
    assert "q is null" in L.flk_last_error().decode()
    assert L.flk_attn_decode(FAKE, FAKE, FAKE, FAKE, 16, 8, 128, 0, FAKE, 1 << 30) == _lib.FLK_ERR_ARG
    assert L.flk_attn_prefill(FAKE, FAKE, FAKE, FAKE, 16, 8, 128, 0, 0, FAKE, 1 << 30) == _lib.FLK_ERR_ARG
    assert L.flk_rmsnorm(FAKE, FAKE, FAKE, 0, 1, 1e-6) == _lib.FLK_ERR_ARG
    assert L.flk_rope(FAKE, FAKE, 1, 1, 127, 0, 0) == _lib.FLK_ERR_ARG
    assert L.flk_rope(FAKE, FAKE, 1, 1, 128, 0, 7) == _lib.FLK_ERR_ARG


def test_workspace_checks():
    L = _lib.lib()
    need = L.flk_workspace_bytes(16, 8, 128, 32832, 0, 1)
    assert need > 0
    assert L.flk_attn_decode(FAKE, FAKE, FAKE, FAKE, 16, 8, 128, 32769, None, 0) == _lib.FLK_ERR_WORKSPACE
    assert L.flk_attn_decode(FAKE, FAKE, FAKE, FAKE, 16, 8, 128, 32769, 0x1000, 16) == _lib.FLK_ERR_WORKSPACE
    # Misaligned workspace.
    assert L.flk_attn_decode(FAKE, FAKE, FAKE, FAKE, 16, 8, 128, 32769, 0x1004,
                             need) == _lib.FLK_ERR_WORKSPACE


def test_workspace_bytes_covers_every_call_in_range():
    # A Layer sizes its workspace once from (maxKeys, maxPrefill); every call it
    # can then make must fit. Checked with the per-call sizing query -- nothing
    # is launched.
    L = _lib.lib()
    for H, Hkv in [(16, 8), (16, 16), (4, 1), (12, 4)]:
        for maxk, maxp in [(2048, 512), (32832, 64), (4096, 2048), (100, 100), (40000, 2048)]:
            ws = L.flk_workspace_bytes(H, Hkv, 128, maxk, maxp, 1)
            # Around whole q tiles (64 rows / group queries) and their multiples.
            for n in sorted({1, 2, 15, 16, 17, 20, 21, 22, 31, 32, 33, 41, 42, 43, 63, 64, 65,
                             127, 128, 129, maxp // 2, maxp}):
                for pos0 in sorted({0, 1, maxk // 3, maxk - 2 * n, maxk - n}):
                    if n < 1 or n > maxp or pos0 < 0 or pos0 + n > maxk:
                        continue
                    need = L.flk_call_workspace_bytes(1, H, Hkv, 128, n, pos0, 1)
                    assert 0 <= need <= ws, (H, Hkv, maxk, maxp, n, pos0)
            for nk in sorted({1, 2, min(511, maxk), maxk // 2, maxk}):
                assert 0 <= L.flk_call_workspace_bytes(0, H, Hkv, 128, nk, 0, 1) <= ws


def test_ragged_workspace_bound():
    L = _lib.lib()
    for seqs in (1, 3, 64, 200):
        ws = L.flk_workspace_bytes(16, 8, 128, 16385, 0, seqs)
        for maxn in (1, 100, 1024, 5000, 16385):
            for s in range(1, seqs + 1, max(1, seqs // 7)):
                assert 0 <= L.flk_call_workspace_bytes(2, 16, 8, 128, maxn, 0, s) <= ws


def test_q8_matvec_guards():
    L = _lib.lib()
    rc, msg = code_and_msg(L.flk_q8_matvec(FAKE, FAKE, FAKE, FAKE, 16, 48, 1))
    assert rc == _lib.FLK_ERR_ARG and "multiple of 32" in msg
    rc, msg = code_and_msg(L.flk_q8_matvec(FAKE, FAKE, FAKE, FAKE, 0, 64, 1))
    assert rc == _lib.FLK_ERR_ARG
    rc, msg = code_and_msg(L.flk_q8_matvec(FAKE, FAKE, FAKE, FAKE, 16, 64, 70000))
    assert rc == _lib.FLK_ERR_UNSUPPORTED
    rc, msg = code_and_msg(L.flk_q8_matvec(FAKE + 4, FAKE, FAKE, FAKE, 16, 64, 1))
    assert rc == _lib.FLK_ERR_ARG and "aligned" in msg
    rc, msg = code_and_msg(L.flk_q8_matvec(None, FAKE, FAKE, FAKE, 16, 64, 1))
    assert rc == _lib.FLK_ERR_ARG and "null" in msg
    # The fused inputs are read as float4s too.
    rc, msg = code_and_msg(L.flk_q8_matvec_ex(FAKE, FAKE, FAKE, FAKE, 16, 64, 8, FAKE + 4, 1e-6,
                                              None, None))
    assert rc == _lib.FLK_ERR_ARG and "norm_gain" in msg and "aligned" in msg
    rc, msg = code_and_msg(L.flk_q8_matvec_ex(FAKE, FAKE, FAKE, FAKE, 16, 64, 8, None, 0.0,
                                              FAKE + 8, None))
    assert rc == _lib.FLK_ERR_ARG and "up" in msg and "aligned" in msg
    rc, msg = code_and_msg(L.flk_q8_gate_up_swiglu(FAKE, FAKE, FAKE, FAKE, 16, 64, 8, FAKE + 12,
                                                   1e-6))
    assert rc == _lib.FLK_ERR_ARG and "norm_gain" in msg and "aligned" in msg


def test_strided_prologue_guards():
    L = _lib.lib()
    args = (FAKE, FAKE, FAKE, 1e-6, 0, FAKE, FAKE, FAKE, 4, 0, 16, 8, 128, 64)
    rc, msg = code_and_msg(L.flk_qk_prologue_strided(FAKE, FAKE, FAKE, 2047, *args))
    assert rc == _lib.FLK_ERR_ARG and "in_stride" in msg
    rc, msg = code_and_msg(L.flk_qk_prologue_strided(FAKE, FAKE, FAKE, 4096, FAKE, FAKE, FAKE, 1e-6,
                                                     0, FAKE, FAKE, FAKE, 4, 62, 16, 8, 128, 64))
    assert rc == _lib.FLK_ERR_CACHE_FULL


def test_q8_split_matches_oracle():
    # Host-side repack (no GPU): the library's splitQ8 against the oracle's.
    import numpy as np
    import oracle
    rng = np.random.default_rng(3)
    rows, cols = 5, 96
    packed = oracle.quant_matrix_q8(rng.normal(0, 0.05, rows * cols), rows, cols)
    qs = np.empty(rows * cols, np.int8)
    sc = np.empty(rows * cols // 32, np.uint16)
    assert _lib.lib().flk_q8_split(packed.ctypes.data, rows, cols, qs.ctypes.data,
                                   sc.ctypes.data) == 0
    want_qs, want_sc = oracle.split_q8(packed, rows, cols)
    assert np.array_equal(qs, want_qs) and np.array_equal(sc, want_sc)


@pytest.mark.parametrize("which", ["q_raw", "k_raw", "v_raw"])
def test_decode_layer_rejects_misaligned_raw_rows(which):
    # The fused layer call reads the raw q, k, v rows as float4s: a pointer
    # off a 16-byte boundary is refused on the host, for both position forms.
    L = _lib.lib()
    raw = {"q_raw": FAKE, "k_raw": FAKE, "v_raw": FAKE}
    raw[which] = FAKE + 4
    rest = (FAKE, FAKE, FAKE, 1e-6, 0, FAKE, FAKE, FAKE, FAKE)
    rc, msg = code_and_msg(L.flk_decode_layer(raw["q_raw"], raw["k_raw"], raw["v_raw"], *rest,
                                              10, 16, 8, 128, 2048, FAKE, 1 << 30))
    assert rc == _lib.FLK_ERR_ARG and which in msg and "aligned" in msg
    rc, msg = code_and_msg(L.flk_decode_layer_dev(raw["q_raw"], raw["k_raw"], raw["v_raw"], *rest,
                                                  FAKE, 16, 8, 128, 2048, FAKE, 1 << 30))
    assert rc == _lib.FLK_ERR_ARG and which in msg and "aligned" in msg


@pytest.mark.parametrize("offs_off,nk_off", [(4, 0), (0, 2)])
def test_ragged_rejects_misaligned_device_arrays(offs_off, nk_off):
    # seq_row_off and n_keys are read as naturally aligned words on the device.
    L = _lib.lib()
    rc, msg = code_and_msg(L.flk_attn_decode_ragged(FAKE, FAKE, FAKE, FAKE + offs_off,
                                                    FAKE + nk_off, FAKE, 4, 100, 16, 8, 128,
                                                    FAKE, 1 << 30))
    assert rc == _lib.FLK_ERR_ARG and "aligned" in msg


def test_decode_layer_dev_rejects_misaligned_key_count():
    L = _lib.lib()
    rc, msg = code_and_msg(L.flk_decode_layer_dev(*([FAKE] * 6), 1e-6, 0, *([FAKE] * 4),
                                                  FAKE + 2, 16, 8, 128, 2048, FAKE, 1 << 30))
    assert rc == _lib.FLK_ERR_ARG and "aligned" in msg


def test_dropped_buffers_are_freed_at_sync_not_on_collection():
    # A DeviceBuffer that is garbage-collected must not call flk_free (which
    # waits for the device) on the spot; its pointer is parked until sync().
    from flock_amd import ops
    b = ops.DeviceBuffer.__new__(ops.DeviceBuffer)  # no allocation: a stand-in pointer
    b.ptr, b.nbytes = FAKE, 4
    before = list(ops._pending_free)
    del b
    assert ops._pending_free == before + [FAKE]
    ops._pending_free.remove(FAKE)


def test_noalloc_decode_rejects_calls_beyond_its_static_scratch():
    # 64 heads of width 128 over 100000 keys need 256 splits x 64 heads x 520
    # B = 8.5 MB of partials, above the 8 MiB static array: refused before any
    # device call (there is no GPU here to reach).
    L = _lib.lib()
    rc, msg = code_and_msg(L.flk_decode_layer_noalloc(*([FAKE] * 6), 1e-6, 0, *([FAKE] * 4),
                                                      99999, 64, 8, 128, 100000))
    assert rc == _lib.FLK_ERR_WORKSPACE and "static scratch" in msg
    rc, msg = code_and_msg(L.flk_decode_layer_noalloc(*([FAKE] * 6), 1e-6, 0, *([FAKE] * 4),
                                                      2048, 16, 8, 128, 2048))
    assert rc == _lib.FLK_ERR_CACHE_FULL


def test_prefill_rejects_rows_too_wide_for_its_tile_offsets():
    # A 64-row key tile is addressed with 32-bit byte offsets: 65536 kv heads
    # of 128 floats make a tile of 2 GiB, which is refused on the host.
    L = _lib.lib()
    rc, msg = code_and_msg(L.flk_attn_prefill(FAKE, FAKE, FAKE, FAKE, 65536, 65536, 128, 4, 0,
                                              FAKE, 1 << 40))
    assert rc == _lib.FLK_ERR_UNSUPPORTED and "2 GiB" in msg
