"""The C-ABI library loads and exports every symbol include/mimg.h declares
(no GPU call: this runs in the CPU suite)."""
import os
import re

from conftest import ROOT


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "mimg.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mimg_\w+)\s*\(", text)))


def test_header_matches_python_signatures():
    import mimg

    assert declared_symbols() == sorted(mimg.SIGNATURES)


def test_library_exports_every_declared_symbol():
    import mimg

    lib = mimg.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_version_and_error_without_gpu_calls():
    import mimg

    lib = mimg.load()
    assert lib.mimg_version() >= 1
    assert lib.mimg_last_error() == b""
    # pure-host helpers that touch no device
    assert lib.mimg_a8_workspace_bytes(1, 4096) > 4096
    assert mimg.a8_workspace_offsets(2, 512)[0] == 0


def test_status_codes_in_header():
    text = open(os.path.join(ROOT, "include", "mimg.h")).read()
    assert "#define MIMG_OK 0" in text and "#define MIMG_NOT_HANDLED 1" in text
