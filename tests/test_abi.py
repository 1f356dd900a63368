"""The C ABI library: it loads without a GPU and exports every function include/spx_sampler.h declares; argument
checks that refuse a call before any device work."""

import ctypes
import os
import re

import pytest

import workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "spx_sampler.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(spx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_exports():
    spx = workloads.spx_module()
    assert declared_functions() == sorted(spx.EXPORTS)


def test_library_exports_every_declared_symbol():
    spx = workloads.spx_module()
    lib = spx.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_params_record_layout():
    spx = workloads.spx_module()
    assert spx.ROW_PARAMS.itemsize == 32
    assert [spx.ROW_PARAMS.fields[n][1] for n in spx.ROW_PARAMS.names] == [0, 4, 8, 12, 16, 20, 24, 28]


def test_refusals_without_a_device():
    spx = workloads.spx_module()
    lib = spx.load_library()
    # A null handle and a null output pointer are refused before any HIP call.
    assert lib.spx_sample_rows(None, None, 0, 1, 10, 10, None, None, None, 0, None, None, None, None, None, None,
                               None, None) == 1
    assert b"handle" in lib.spx_last_error()
    assert lib.spx_sampler_create(None, 1, 1, 0, 0) == 1
    h = ctypes.c_void_p()
    assert lib.spx_sampler_create(ctypes.byref(h), 0, 10, 0, 0) == 1
    assert lib.spx_argmax_rows(None, None, 0, 1, 10, 10, None, 0, None, None) == 1


def test_missing_library_fails_loudly(tmp_path):
    spx = workloads.spx_module()
    saved = spx._lib
    spx._lib = None
    try:
        with pytest.raises(RuntimeError, match="not built"):
            spx.load_library(str(tmp_path / "absent.so"))
    finally:
        spx._lib = saved


def test_refusals_of_the_family_entries_without_a_device():
    # Each refusal returns before any HIP call: DRY settings whose window or penalties the device cannot hold, ids
    # outside the vocabulary, a head pick without a handle or with a hidden size the product does not take, and a
    # no-alloc call past its static workspace.
    spx = workloads.spx_module()
    lib = spx.load_library()
    ok = spx.DryConfig(0.8, 1.75, 3.0, 2, 64, 8, 0)
    ex = (ctypes.c_int32 * 3)(0, 1, 2)
    assert lib.spx_dry_update_rows(1, None, ex, 3, None, None, None, 73, None) == 1
    assert lib.spx_dry_update_rows(1, ctypes.byref(ok), ex, 3, None, None, None, 72, None) == 1  # window of 73
    assert b"hist_stride" in lib.spx_last_error()
    assert lib.spx_dry_update_rows(1, ctypes.byref(ok), ex, 9, None, None, None, 73, None) == 1
    # penalties that fall with the length never reach max_penalty: past 128 lengths the table cannot end
    falling = spx.DryConfig(0.8, 0.5, 3.0, 2, 64, 400, 0)
    assert lib.spx_dry_update_rows(1, ctypes.byref(falling), ex, 3, None, None, None, 465, None) == 1
    assert b"max_penalty" in lib.spx_last_error()
    # ... while rising ones that reach it do not need the table's end
    rising = spx.DryConfig(0.8, 1.75, 3.0, 2, 64, 400, 0)
    assert lib.spx_dry_update_rows(0, ctypes.byref(rising), ex, 3, None, None, None, 465, None) == 0
    assert lib.spx_haru_shape_rows(None, 1, 100, 100, ctypes.byref(ok), ex, 3, None, None, 73, None, 0, 1, 100, 0.0,
                                   None, None, None, None, 0, None) == 1
    assert lib.spx_head_argmax_rows(None, None, 2048, None, 1e-6, None, 2048, 1, 2048, 151936, None, None, None) == 1
    assert b"handle" in lib.spx_last_error()
    args = [None, spx.F32, 4096, 3072, 3072, None, None, 0, None, 0, None, None, None, None, None, None, None, 0, None]
    assert lib.spx_sample_rows_noalloc(*args) == 1
    assert b"SPX_NOALLOC_MAX_ROWS" in lib.spx_last_error()
