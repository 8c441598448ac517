"""The C-ABI library loads on a host without a GPU, exports every entry
point declared in include/*.h, and its host-only generators match the oracle
bit for bit."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

import jade_hip
import oracle_binding as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for header in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for match in re.finditer(r"\b(?:int|void|uint32_t)\s+(\w+)\s*\(", text):
            names.add(match.group(1))
    return sorted(names)


def test_headers_declare_the_reference_entry_points():
    names = set(declared_functions())
    # native/jade_runtime_corex.h:18-31 and native/jade_corex.h:17-29.
    for name in ["jr_version", "jr_create", "jr_destroy", "jr_info", "jr_alloc", "jr_free", "jr_upload",
                 "jr_download", "jr_execute", "jade_corex_abi_version", "jade_corex_create", "jade_corex_upload",
                 "jade_corex_run", "jade_corex_download", "jade_corex_device_info", "jade_corex_destroy"]:
        assert name in names


@pytest.mark.parametrize("name", declared_functions())
def test_library_exports_declared_symbol(name):
    lib = ctypes.CDLL(jade_hip.LIBRARY_PATH)
    assert hasattr(lib, name)


def test_abi_versions():
    lib = jade_hip.load()
    assert lib.jr_version() == 2
    assert lib.jade_corex_abi_version() == 1


def test_fill_values_matches_oracle_bit_for_bit():
    for seed, scale in [(0x1234, 1.0), (0x3333, 1.0 / 32.0), (0x12345678, 1.0), (0x9ABCDEF1, 1.0), (7, 2.0)]:
        np.testing.assert_array_equal(jade_hip.fill_values(4099, seed, scale), orc.values(4099, seed, scale))


def test_fill_normal_matches_oracle_bit_for_bit():
    for seed, mean, sigma in [(0x1111, 0.0, 1.0), (0x4444, 0.0, 0.02), (0x7777, 1.0, 0.5), (9, 0.0, 2.0)]:
        np.testing.assert_array_equal(jade_hip.fill_normal(4099, seed, mean, sigma), orc.normal(4099, seed, mean,
                                                                                                  sigma))


def test_null_and_unknown_handles_are_rejected_without_a_device():
    lib = jade_hip.load()
    err = ctypes.create_string_buffer(1024)
    out = ctypes.c_void_p()
    assert lib.jr_alloc(None, 16, ctypes.byref(out), err, 1024) == 1
    assert b"context" in err.value
    assert lib.jr_alloc(ctypes.c_void_p(0x1234), 16, ctypes.byref(out), err, 1024) == 1
    assert lib.jr_create(-1, ctypes.byref(out), err, 1024) == 1
    assert lib.jr_execute_dispatches(None, None, 0, 1, None, err, 1024) == 1
    assert lib.jade_corex_create(0, 1, 1, 0, 0, ctypes.byref(out), err, 1024) == 1
    assert lib.jade_corex_create(1, 1, 1, 0, 1, ctypes.byref(out), err, 1024) == 1  # FP16 mode not provided
    assert b"precision" in err.value
    lib.jr_destroy(None)
    lib.jr_free(None, None)
    lib.jade_corex_destroy(None)


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="host has a GPU")
def test_create_without_a_gpu_fails_cleanly():
    with pytest.raises(jade_hip.JadeError) as info:
        jade_hip.HipRuntime(0)
    assert info.value.code in (1, 2)
