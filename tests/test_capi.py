"""C-ABI checks that need no GPU: the library loads, exports exactly what
include/verace_sssd.h declares, and rejects bad arguments before touching the device."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "verace_sssd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(vmi_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from verace_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libverace_sssd.so is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declarations_are_exported(lib):
    from verace_amd import _lib
    decl = _declared()
    assert decl == sorted(_lib.EXPORTED)
    for name in decl:
        assert hasattr(lib, name), name


def test_exported_symbols_match_nm():
    import subprocess
    from verace_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(set(re.findall(r" T (vmi_\w+)", out)))
    assert exported == _declared()


def test_version_and_status_strings(lib):
    assert lib.vmi_version() >= 100
    assert lib.vmi_status_string(0) == b"ok"
    assert b"workspace" in lib.vmi_status_string(3)


def test_workspace_query(lib):
    n = ctypes.c_size_t(123)
    assert lib.vmi_sssd_scan_workspace_bytes(8, 4096, 8, 128, 1, ctypes.byref(n)) == 0
    assert lib.vmi_sssd_scan_workspace_bytes(1, 1, 1, 0, 1, ctypes.byref(n)) == 1
    assert lib.vmi_sssd_scan_workspace_bytes(1, 1, 1, 16, 7, ctypes.byref(n)) == 1
    assert lib.vmi_cham_ns_workspace_bytes(2, 16, ctypes.byref(n)) == 0
    assert n.value == 6 * 2 * 16 * 16 * 4
    # CHAM scan: h <= 128 keeps a state per 16 tokens after the first chunk; larger h a
    # readout snapshot per 64 tokens (rows padded to 256/512/1024) plus the coefficient,
    # Z and initial-retraction pieces; h > 1024 is not built
    assert lib.vmi_cham_scan_workspace_bytes(2, 48, 128, ctypes.byref(n)) == 0
    assert n.value == 2 * 2 * 2 * 128 * 128 * 4
    assert lib.vmi_cham_scan_workspace_bytes(1, 64, 1024, ctypes.byref(n)) == 0
    assert n.value >= (2 * 1024 * 1024 + 2 * 64 * 1024 + 8 * 1024 * 1024) * 4
    assert lib.vmi_cham_scan_workspace_bytes(1, 64, 1025, ctypes.byref(n)) == 2


def test_argument_errors_before_any_device_call(lib):
    # null pointers / bad sizes are rejected on the host (no HIP call is made)
    assert lib.vmi_sssd_scan_fwd(None, None, None, None, 1, 1, None, None, None,
                                 1, 4, 1, 16, None, 0, None) == 1
    assert lib.vmi_sssd_scan_fwd(None, None, None, None, 9, 1, None, None, None,
                                 1, 4, 1, 16, None, 0, None) == 1
    big = ctypes.c_void_p(0x1000)
    assert lib.vmi_sssd_scan_fwd(big, big, big, big, 1, 1, None, None, big,
                                 1, 4, 1, 512, None, 0, None) == 2
    # psi_out overlapping psi_in is forbidden for the scan
    assert lib.vmi_sssd_scan_fwd(big, big, big, big, 1, 1, big, None, big,
                                 1, 4, 1, 16, None, 0, None) == 4
    assert lib.vmi_sssd_step_inplace(None, None, None, None, 1, 1, None, None, 1, 1, 16, None) == 1
    assert lib.vmi_sssd_step_slots(None, None, None, None, 1, 1, None, 4, None, None, None,
                                   1, 1, 16, None) == 1
    assert lib.vmi_sssd_step_slots(big, big, big, big, 1, 1, big, -1, big, big, big,
                                   1, 1, 16, None) == 1
    assert lib.vmi_sssd_step_slots(big, big, big, big, 1, 1, big, 4, big, big, big,
                                   1, 1, 512, None) == 2
    # an empty batch is a no-op that touches nothing
    assert lib.vmi_sssd_step_slots(None, None, None, None, 1, 1, None, 0, None, None, None,
                                   0, 8, 128, None) == 0
    assert lib.vmi_cham_ns_retraction(None, None, None, None, 1, 4, 3, None, 0, None) == 1
