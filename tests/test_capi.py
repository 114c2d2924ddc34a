"""CPU-side checks of the boundary: the C-ABI library loads, exports every entry point
that include/pd_mi355x.h declares, the Python binding covers exactly those, the host key
derivation matches the oracle, and the product path fails loudly without the library."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pd_mi355x.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pd_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = header_symbols()
    assert "pd_dense_step" in syms and "pd_grouped_gemm_dw" in syms and len(syms) >= 25


def test_library_exports_every_declared_symbol():
    from param_decomp_amd import _lib as L

    if not os.path.exists(L.LIB_PATH):
        pytest.skip("HIP library not built")
    lib = ctypes.CDLL(L.LIB_PATH)
    missing = [s for s in header_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_the_header():
    from param_decomp_amd import _lib as L

    assert sorted(L.exported_symbols()) == header_symbols()


def _header_arities():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"\b(pd_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_binding_arity_matches_the_header():
    """Every ctypes signature has exactly the header's parameter count: an argument past
    the declared argtypes would go through ctypes' variadic conversion (a 32-bit int in a
    64-bit slot), which corrupts pointer arguments such as the stream."""
    from param_decomp_amd import _lib as L

    ar = _header_arities()
    bad = {n: (ar.get(n), len(args)) for n, (_, args) in L._SIGNATURES.items() if ar.get(n) != len(args)}
    assert not bad, bad


def test_missing_library_raises(monkeypatch, tmp_path):
    from param_decomp_amd import _lib as L

    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(L.PDError, match="not built"):
        L.load()


def test_cpu_tensors_are_rejected():
    import torch

    from param_decomp_amd import _lib as L

    with pytest.raises(L.PDError, match="GPU tensors"):
        L.ptr(torch.zeros(3))


def test_host_prng_matches_oracle():
    from oracle import threefry as tf
    from param_decomp_amd import prng

    for seed in (0, 3, 2**31 + 5):
        k = prng.PRNGKey(seed)
        assert prng.split(k, 4) == tf.split(tf.prng_key(seed), 4)
        assert prng.split(k, 4, partitionable=False) == tf.split(tf.prng_key(seed), 4, partitionable=False)
        assert prng.fold_in(k, 12) == tf.fold_in(tf.prng_key(seed), 12)
        assert prng.threefry2x32((0, 0), 0, 0) == (0x6B200159, 0x99BA4EFE)
