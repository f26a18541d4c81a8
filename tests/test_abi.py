"""The C-ABI library loads, exports every symbol the header declares, and validates on the host."""
import ctypes
import os
import re

import pytest

import li_sparse._lib as L

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "li_sparse_attn.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(li_\w+)\s*\(", text, flags=re.M)))


def test_every_declared_symbol_is_exported():
    syms = declared_symbols()
    assert len(syms) >= 7
    for s in syms:
        assert hasattr(L.lib, s), s
    assert set(syms) == set(L.SIGNATURES), "ctypes signatures and header disagree"


def test_version_and_status_strings():
    assert L.lib.li_abi_version() == L.ABI_VERSION
    assert L.status_string(L.LI_ERR_INDEX_RANGE) == "Sparse indices out of bounds."
    assert L.status_string(L.LI_OK) == "ok"
    assert L.status_string(123) == "unknown status"


def _strides(*v):
    return L.i64_array(v)


def test_host_validation_needs_no_gpu():
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    s4, s3 = _strides(1, 1, 1, 1), _strides(1, 1, 1)
    bsa = L.lib.li_bsa_fwd
    # K length not a multiple of the block size
    assert bsa(0, 1, 1, 128, 200, 128, fake, fake, fake, fake, s4, 1, fake, s3, 1.0, 128, fake, None, None, 0, 0, None) == L.LI_ERR_K_LEN
    # no key block at all (Lk = 0), on the bf16 and the e4m3 tiled entry points
    assert bsa(0, 1, 1, 128, 0, 128, fake, fake, fake, fake, s4, 1, fake, s3, 1.0, 128, fake, None, None, 0, 0, None) == L.LI_ERR_SHAPE
    assert L.lib.li_bsa_fwd_fp8(1, 1, 128, 0, 128, fake, fake, fake, fake, fake, fake, s4, 1, fake, s3, 1.0, 128, fake,
                                None, None, 0, 0, None) == L.LI_ERR_SHAPE
    # null pointers
    assert bsa(0, 1, 1, 128, 256, 128, None, fake, fake, fake, s4, 1, fake, s3, 1.0, 128, fake, None, None, 0, 0, None) == L.LI_ERR_INVALID_ARG
    # unsupported head dim / block size / dtype
    assert bsa(0, 1, 1, 128, 256, 96, fake, fake, fake, fake, s4, 1, fake, s3, 1.0, 128, fake, None, None, 0, 0, None) == L.LI_ERR_UNSUPPORTED
    assert bsa(0, 1, 1, 128, 256, 128, fake, fake, fake, fake, s4, 1, fake, s3, 1.0, 32, fake, None, None, 0, 0, None) == L.LI_ERR_UNSUPPORTED
    assert bsa(7, 1, 1, 128, 256, 128, fake, fake, fake, fake, s4, 1, fake, s3, 1.0, 128, fake, None, None, 0, 0, None) == L.LI_ERR_UNSUPPORTED
    # misaligned pointers
    odd = ctypes.c_void_p(18)
    assert bsa(0, 1, 1, 128, 256, 128, odd, fake, fake, fake, s4, 1, fake, s3, 1.0, 128, fake, None, None, 0, 0, None) == L.LI_ERR_INVALID_ARG
    # tile geometry with a wrong nh
    g = L.TileGeom(2, 30, 52, 2, 8, 8, 3, 7)
    assert L.lib.li_q_prep(0, 1, 1, 128, fake, s4, fake, _strides(1, 1, 1, 1, 1), fake, s4, ctypes.byref(g),
                           None) == L.LI_ERR_SHAPE
    g = L.TileGeom(2, 30, 52, 2, 8, 8, 4, 7)
    assert L.lib.li_untile(0, 1, 1, 100, fake, _strides(1, 1, 1, 1, 1), fake, s4, ctypes.byref(g),
                           None) == L.LI_ERR_UNSUPPORTED
    # mask builder limits
    p = L.MaskParams(metric=1, budget_mode=0, topk_ratio=0.3, min_budget=7, nq=4, nk=20000, nh=4, nw=7, kmax=10)
    assert L.lib.li_block_mask(0, 1, 1, 128, fake, s4, fake, s4, ctypes.byref(p), fake, fake, None,
                               None) == L.LI_ERR_TOO_LARGE
    p = L.MaskParams(metric=9, budget_mode=0, topk_ratio=0.3, nq=4, nk=20, nh=4, nw=7, kmax=10)
    assert L.lib.li_block_mask(0, 1, 1, 128, fake, s4, fake, s4, ctypes.byref(p), fake, fake, None,
                               None) == L.LI_ERR_INVALID_ARG


def test_oracle_is_not_imported_by_the_product():
    import sys

    pkg = os.path.dirname(L.__file__)
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(root, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle", src, flags=re.M), f
    assert "oracle" not in {m.split(".")[0] for m in sys.modules if m.startswith("li_sparse")}


def test_single_hip_runtime_is_mapped():
    # The library must bind to the HIP runtime torch loaded (one libamdhip64 in the process);
    # two runtimes would make torch's streams and pointers foreign to the library's launches.
    import torch  # noqa: F401

    maps = open("/proc/self/maps").read()
    libs = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(libs) == 1, libs
    ours = os.path.realpath(L.LIB_PATH)
    assert any(os.path.realpath(line.split()[-1]) == ours for line in maps.splitlines() if "libli_sparse" in line)
