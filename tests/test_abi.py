"""CPU checks of the C-ABI boundary: the shared library loads, exports exactly what
include/moe_ffn.h declares, and rejects bad arguments on the host (no kernel runs)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "moe_ffn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


def test_header_matches_binding_list(pkg):
    assert declared_functions() == sorted(pkg.EXPORTS)


def test_library_exports_every_declared_symbol(pkg):
    L = pkg.lib()
    missing = [f for f in declared_functions() if not hasattr(L, f)]
    assert not missing, missing
    out = os.popen(f"nm -D --defined-only {pkg.LIB_PATH}").read()
    exported = set(re.findall(r"\bT (moe_[a-z0-9_]+)", out))
    assert set(declared_functions()) <= exported


def test_library_is_gfx950(pkg):
    blob = open(pkg.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_host_validation_without_gpu(pkg):
    L = pkg.lib()
    vp = ctypes.c_void_p
    # null context / pointers -> MOE_EINVAL, message set
    assert L.moe_ffn(None, 0, None, None, None, 1, None, 0, None) == pkg.MOE_EINVAL
    assert b"null" in L.moe_last_error()
    assert L.moe_destroy(None) == pkg.MOE_EINVAL
    assert L.moe_router_topk(None, None, 1, None, None, None) == pkg.MOE_EINVAL
    assert L.moe_bucket_fill(None, None, None, 1, None, None, None, None) == pkg.MOE_EINVAL
    assert L.moe_dequant_iq4xs(None, 1, None, None) == pkg.MOE_EINVAL
    assert L.moe_bind_layer(None, 0, None) == pkg.MOE_EINVAL
    assert L.moe_create(0, None, ctypes.byref(vp())) == pkg.MOE_EINVAL
    # shape that is not compiled -> MOE_EUNSUPPORTED before any HIP call
    cfg = pkg._Config(4096, 512, 256, 1, 16, 0)
    h = vp()
    assert L.moe_create(0, ctypes.byref(cfg), ctypes.byref(h)) == pkg.MOE_EUNSUPPORTED
    assert b"not compiled" in L.moe_last_error()
    for bad in [pkg._Config(2048, 512, 4, 1, 16, 0), pkg._Config(2048, 512, 257, 1, 16, 0),
                pkg._Config(2048, 512, 1024, 1, 16, 0), pkg._Config(2048, 512, 256, 0, 16, 0),
                pkg._Config(2048, 512, 256, 1, 0, 0), pkg._Config(2048, 512, 256, 1, 70000, 0),
                pkg._Config(2048, 512, 256, 1, 16, 7)]:
        assert L.moe_create(0, ctypes.byref(bad), ctypes.byref(h)) == pkg.MOE_EINVAL
    assert L.moe_gen_logits(None, 1, 256, 0, 0, 0.0, 0.0, None) == pkg.MOE_EINVAL
    # misaligned dequant buffers are refused on the host
    assert L.moe_dequant_iq4xs(ctypes.c_void_p(0x1004), 1, ctypes.c_void_p(0x2000), None) == pkg.MOE_EINVAL


def test_oracle_is_not_linked_by_product(pkg):
    # The product library must not reference the oracle in any form.
    blob = open(pkg.LIB_PATH, "rb").read()
    assert b"orc_" not in blob and b"liborc" not in blob
    for root, _, files in os.walk(os.path.join(ROOT, "moe-680m_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                text = open(os.path.join(root, f), errors="replace").read()
                assert "oracle" not in text.replace("no oracle", ""), f
