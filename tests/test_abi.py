"""The C-ABI library loads, exports exactly what include/needle_hip.h
declares, and fails cleanly before nh_init (no GPU needed)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import needle_hip
import oracle as o

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "needle_hip.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(nh_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared()
    assert len(names) >= 20
    assert set(names) == set(needle_hip.SIGNATURES), set(names) ^ set(needle_hip.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = needle_hip.load_library()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.nh_version() == 101


def test_calls_before_init_fail_cleanly():
    lib = needle_hip.load_library()
    h = C.c_void_p()
    packed = np.zeros(64, np.uint8)
    norms = np.zeros(1, np.uint16)
    rc = lib.nh_qmat_from_cq(packed.ctypes.data_as(C.c_void_p), 64, norms.ctypes.data_as(C.c_void_p), 1, 1, 128, 4,
                             128, C.byref(h))
    assert rc == -5
    assert b"nh_init" in lib.nh_last_error()
    a = C.c_void_p()
    assert lib.nh_qact_new(1, 128, 4, C.byref(a)) == -5
    assert lib.nh_matmul(None, None, None, 0, 0, None) == -5


def test_host_generator_matches_oracle():
    # The product's seeded-input generator against the oracle's restatement
    # of crates/needle-train/src/rand.rs:161-217 (itself pinned by the
    # reference's KATs).
    k = [0, 0]
    for _ in range(3):
        k2, sub = needle_hip.split(k)
        assert (k2, sub) == o.split(k)
        got = needle_hip.normal(sub, 100_003)
        want = o.normal(sub, 100_003)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        k = k2


def test_kernel_sources_have_no_packed_fp32_or_scalar_stores():
    # Hand-written kernels use no packed-FP32 instructions.
    src = os.path.join(os.path.dirname(HEADER), "..", "needle-rs_amd", "csrc")
    for f in os.listdir(src):
        text = open(os.path.join(src, f)).read()
        assert "v_pk_" not in text, f
