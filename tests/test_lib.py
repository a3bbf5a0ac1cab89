"""The C-ABI library loads and exports every symbol include/*.h declares (no compute)."""
import glob
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER_DECL = re.compile(r"CSDR_API\s+[^;(]*?\b((?:csdr|cortex)_\w+)\s*\(", re.S)


def declared_symbols() -> set[str]:
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        names |= set(HEADER_DECL.findall(open(h).read()))
    return names


def test_header_declares_entry_points():
    names = declared_symbols()
    assert {"csdr_hsdb_load", "csdr_hsdb_matmul", "csdr_hsdb_decompress",
            "cortex_inference_engine_create", "cortex_inference_engine_run_layer",
            "csdr_archive_open", "csdr_hsda_load", "csdr_decoder_generate"} <= names


def test_library_exports_every_declared_symbol():
    from cortexsdr_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libcortexsdr_amd.so not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = declared_symbols() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    # the Python binding knows every declared symbol too
    assert declared_symbols() <= set(_lib.exported_symbols())


def test_library_loads_with_one_hip_runtime():
    from cortexsdr_amd import _lib

    lib = _lib.load()
    assert lib.csdr_version().decode().startswith("cortexsdr_amd")
    assert len(_lib._hip_runtimes_mapped()) <= 1


def test_product_does_not_reference_oracle():
    # the product package never imports or loads the checker
    for path in glob.glob(os.path.join(ROOT, "cortexsdr_amd", "**", "*.*"), recursive=True):
        if path.endswith((".py", ".hip", ".cpp", ".hpp", ".h")):
            text = open(path).read()
            assert "import oracle" not in text and "liborc" not in text, path
            assert "csdr_oracle" not in text and "libcsdr_ref" not in text, path
