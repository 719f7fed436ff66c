"""CPU checks of the C ABI: the library loads and exports every declared symbol."""
import ctypes
import os
import re

import pytest

import sharpmind_amd
from sharpmind_amd import _abi

HEADER = os.path.join(os.path.dirname(__file__), "..", "include", "sharpmind_hip.h")


def test_header_parses_to_prototypes():
    protos = _abi.prototypes(HEADER)
    names = [p[0] for p in protos]
    assert len(names) == len(set(names))
    declared = set(re.findall(r"\b(smhip_\w+)\s*\(", re.sub(r"/\*.*?\*/", " ", open(HEADER).read(), flags=re.S)))
    assert declared == set(names)


def test_library_exports_every_declared_symbol():
    lib = sharpmind_amd.lib()
    missing = [n for n, _, _ in _abi.prototypes(HEADER) if not hasattr(lib, n)]
    assert not missing, missing


def test_runtime_queries_without_gpu():
    lib = sharpmind_amd.lib()
    assert lib.smhip_version() >= 100
    assert lib.smhip_device_count() >= 0


def test_argument_validation_reports_error():
    lib = sharpmind_amd.lib()
    rc = lib.smhip_grad_rmsnorm(None, None, None, None, None, None, 4, 0, None)
    assert rc == -1
    assert b"bad shape" in lib.smhip_last_error()
    with pytest.raises(sharpmind_amd.SmHipError):
        sharpmind_amd.check(rc)


def test_rope_tables_match_oracle():
    """Host-side table builder of the library equals the oracle's restatement of RoPE.cs:99-148."""
    import numpy as np
    import oracle
    from sharpmind_amd import hip
    for theta, D in ((1e4, 64), (1e6, 128)):
        c, s = hip.rope_tables(theta, D, 300)
        oc = np.zeros_like(c)
        os_ = np.zeros_like(s)
        oracle.lib().orc_rope_tables(theta, D, 300, oc, os_)
        assert (c == oc).all() and (s == os_).all()
