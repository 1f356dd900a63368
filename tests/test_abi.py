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
