"""The C ABI as shipped: libperegrine_hip.so loads on a host without a GPU and
exports every function include/peregrine_hip.h declares; the Python binding
declares exactly that set. No compute call is made."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "peregrine_hip.h")
LIB = os.path.join(ROOT, "peregrine_amd", "libperegrine_hip.so")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(coli_hip_\w+)\s*\(", text))


def test_header_declares_the_reference_surface():
    """Every function of the reference C ABI bound from Rust
    (crates/peregrine-cuda/src/lib.rs:40-109) has its coli_hip_ counterpart."""
    names = header_functions()
    ref = ["init", "shutdown", "device_count", "probe_device_count", "mem_info", "tensor_upload", "tensor_free",
           "expert_group", "group_stats", "graph_begin", "graph_end", "graph_launch", "graph_free",
           "expert_group_tiled", "expert_group_reduce", "graph_cache_stats"]
    missing = [n for n in ref if "coli_hip_" + n not in names]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="libperegrine_hip.so not built (run __graft_entry__.build())")
def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in sorted(header_functions()) if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (coli_hip_\w+)$", out, flags=re.M))
    assert exported == header_functions(), (sorted(exported - header_functions()),
                                             sorted(header_functions() - exported))


@pytest.mark.skipif(not os.path.exists(LIB), reason="libperegrine_hip.so not built (run __graft_entry__.build())")
def test_python_binding_declares_the_header():
    from peregrine_amd import _lib
    assert set(_lib.SIGNATURES) == header_functions()


@pytest.mark.skipif(not os.path.exists(LIB), reason="libperegrine_hip.so not built (run __graft_entry__.build())")
def test_library_does_not_link_the_oracle():
    out = subprocess.run(["ldd", LIB], capture_output=True, text=True).stdout
    assert "oracle" not in out
    dyn = subprocess.run(["nm", "-D", LIB], capture_output=True, text=True, check=True).stdout
    assert "orc_" not in dyn
