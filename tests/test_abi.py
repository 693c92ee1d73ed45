"""The C-ABI library loads and exports exactly what include/*.h declares, with
the reference's symbol set as a subset (CPU only: no compute calls)."""
import ctypes
import glob
import os
import re

import pytest

from conftest import ROOT

# The reference C-ABI (split_manifold_lut_experiment/native/include/
# ojasx_lut_c_api.h:40-150): 21 symbols.
REFERENCE_SYMBOLS = [
    "ojasx_get_version", "ojasx_get_backend_name", "ojasx_create_linear",
    "ojasx_set_linear_outliers", "ojasx_linear_forward", "ojasx_get_compressed_size",
    "ojasx_get_dense_size", "ojasx_get_lut_sram_size", "ojasx_get_compression_ratio",
    "ojasx_destroy_linear", "ojasx_create_kv_cache", "ojasx_kv_cache_append",
    "ojasx_kv_cache_attention", "ojasx_kv_cache_get_memory_size",
    "ojasx_kv_cache_get_compression_ratio", "ojasx_destroy_kv_cache", "ojasx_create_moe",
    "ojasx_moe_forward", "ojasx_moe_get_compressed_size", "ojasx_moe_get_compression_ratio",
    "ojasx_destroy_moe",
]


def declared_symbols():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        names += re.findall(r"OJASX_API\s+[^;(]*?\b(ojasx_\w+)\s*\(", src)
    return sorted(set(names))


def test_header_declares_reference_set():
    decl = declared_symbols()
    for s in REFERENCE_SYMBOLS:
        assert s in decl, s


def test_library_exports_every_declared_symbol(pkg):
    L = ctypes.CDLL(pkg._lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing


def test_python_signatures_cover_header(pkg):
    assert sorted(pkg._lib.SIGNATURES) == declared_symbols()


def test_metadata_without_gpu(pkg):
    L = pkg.lib()
    assert L.ojasx_get_version()
    assert b"gfx950" in L.ojasx_get_backend_name()
    # null handles are rejected / report zero without touching the device
    assert L.ojasx_get_compressed_size(None) == 0
    assert L.ojasx_get_compression_ratio(None) == 0.0
    assert L.ojasx_moe_get_compressed_size(None) == 0
    assert L.ojasx_kv_cache_get_memory_size(None) == 0
    assert L.ojasx_linear_forward(None, None, None, 1, 0) == -1
    assert L.ojasx_kv_cache_append(None, 0, None, None) == -1
    assert L.ojasx_moe_forward(None, None, None, None, None, 1) == -1


def test_library_has_gfx950_code_object(pkg):
    data = open(pkg._lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_bench_and_entry_compile_and_refuse_several_gpus():
    """bench.py and __graft_entry__.py parse, and bench.py --gpus 2 exits with
    its one-GPU message before touching torch or a device."""
    import py_compile
    import subprocess
    import sys
    for f in ("bench.py", "__graft_entry__.py"):
        py_compile.compile(os.path.join(ROOT, f), doraise=True)
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert p.returncode == 2
    assert "measures one GPU" in p.stderr
