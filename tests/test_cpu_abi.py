"""The C-ABI library loads on the CPU host and exports every declared symbol
(no compute calls: this container has no GPU)."""
import os
import re

from flashquest_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "fq_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(fq_\w+)\(", text, re.M)))


def test_header_declares_the_python_binding_table():
    assert _declared() == sorted(_lib.SIGNATURES)


def test_library_loads_and_exports_all_symbols():
    lib = _lib.load_library()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.fq_abi_version() == 1


def test_workspace_size_is_pure_host_arithmetic():
    lib = _lib.load_library()
    c = _lib.Int4Cache()
    c.L, c.B, c.H_kv, c.P, c.D = 28, 1, 8, 512, 128
    n = lib.fq_workspace_bytes(c, 24)
    assert n > 28 * 8 * 512 * 4
    assert lib.fq_workspace_bytes(c, 25) == 0


def test_probe_library_is_separate_and_exports_its_entries():
    """The benchmark's measurement probes live in libfq_probe.so with their own
    header (csrc/fq_probe.h), not in the product library or its public header."""
    from flashquest_amd import _probe
    text = open(os.path.join(ROOT, "flashquest_amd", "csrc", "fq_probe.h")).read()
    names = sorted(set(re.findall(r"^\s*int\s+(fq_\w+)\(", text, re.M)))
    assert names == sorted(_probe.SIGNATURES) == ["fq_read_decode_pages", "fq_read_stream"]
    lib = _probe.probe_lib()
    for n in names:
        assert hasattr(lib, n)
        assert not hasattr(_lib.load_library(), n), n
        assert n not in _declared()
    # a refused call reports through the product library's fq_last_error
    assert lib.fq_read_stream(None, 16, None, None) == _lib.FQ_ERR_INVALID
    assert "NULL buffer" in _lib.lib().fq_last_error().decode()
