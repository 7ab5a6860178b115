"""The C-ABI library loads and exports every entry point include/prism_bsa.h
declares, with a binding for each (no compute: runs without a GPU)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "prism_bsa.h")
LIB = os.path.join(ROOT, "prism_amd", "libprism_bsa.so")


def declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(prism_[a-z0-9_]+)\s*\(", txt)))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return sorted(set(l.split()[-1] for l in out.splitlines() if " T prism_" in l))


@pytest.fixture(scope="module", autouse=True)
def built():
    if not os.path.exists(LIB):
        # by file path: importing the package would load the library first
        import importlib.util
        spec = importlib.util.spec_from_file_location("_prism_amd_build", os.path.join(ROOT, "prism_amd", "build.py"))
        build = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(build)
        build.build()


def test_header_declares_entry_points():
    names = declared()
    assert len(names) >= 20
    assert "prism_bsa_fwd" in names and "prism_select_tiles" in names


def test_library_exports_every_declared_symbol():
    missing = set(declared()) - set(exported())
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_every_export_is_declared():
    extra = set(exported()) - set(declared())
    assert not extra, f"exported but not declared in the header: {sorted(extra)}"


def test_ctypes_binding_covers_header():
    from prism_amd import _lib
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name)
        if name not in ("prism_last_error", "prism_abi_version"):
            assert name in _lib.SIGNATURES, f"no ctypes signature for {name}"


def test_binding_arity_matches_header():
    """Each ctypes signature has as many arguments as the header prototype."""
    from prism_amd import _lib
    txt = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, args in _lib.SIGNATURES.items():
        m = re.search(r"\b" + name + r"\s*\(([^)]*)\)", txt)
        assert m, name
        n = len([a for a in m.group(1).split(",") if a.strip()])
        assert n == len(args), (name, n, len(args))


def test_invalid_arguments_raise_without_gpu():
    """Argument validation happens on the host before any launch."""
    from prism_amd import _lib
    with pytest.raises(ValueError, match="multiples of 8"):
        _lib.call("prism_zone_stats", 1, 0, 1, 64, 64, None, 4, 4, 4, 4, 4, 4, 1, 1, None)
    with pytest.raises(ValueError, match="must fit the zone grid"):
        _lib.call("prism_gather_pool", 1, 0, 1, 1, 9 * 8 * 8, 64, None, 1, 1, 8, 8, 8, 9, 8, 8, 0,
                  None, None, None, None, None, None, None, None)
    with pytest.raises(ValueError, match="Tin\\*Hin\\*Win != S"):
        _lib.call("prism_scatter_rows", 1, 1, 1, 500, 64, 1, 8, 8, 8, 7, 8, 8, 1, 0, None)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("prism_bsa_fwd", None, None, None, 1, 128, 128, 64, None, None, None, None, None, None, 0.1, None,
                  None, None, None)
    with pytest.raises(ValueError, match="head_dim"):
        _lib.call("prism_bsa_fwd", 1, 1, 1, 1, 128, 128, 96, None, 1, 1, 1, None, None, 0.1, 1, 1, None, None)
    with pytest.raises(ValueError, match="multiples of 128"):
        _lib.call("prism_bsa_bwd_dq", 1, 1, 1, 1, 1, 1, 1, 128, 192, 64, None, 1, 1, 1, None, None, 0.1, 1, None,
                  None)
    with pytest.raises(ValueError, match="tail must be"):
        _lib.call("prism_pair_order", 1, 100, 64, 101, 1, None)
    with pytest.raises(ValueError, match="group"):
        _lib.call("prism_pair_order", 1, 100, 16, 10, 1, None)
    with pytest.raises(ValueError, match="even row_tiles"):
        _lib.call("prism_pair_tiles", 1, 1, 1, 10, 5, 5, 1, None)
    with pytest.raises(ValueError, match="64 or 128"):
        _lib.call("prism_chunk_gather_pool", 1, 1, 1, 1, 64, None, 4, 4, 4, 4, 4, 4, 2, 2, 2, 128,
                  None, None, None, None, None, None, None, None)
    with pytest.raises(ValueError, match="multiple of the chunk|multiples of the chunk"):
        _lib.call("prism_chunk_scatter_rows", 1, 1, 1, 64, 4, 4, 4, 4, 4, 6, 4, 4, 4, 128, 1, 1, None)
    assert _lib.load().prism_abi_version() == 10
