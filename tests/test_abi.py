"""CPU checks of the C-ABI library: it loads, and exports exactly what include/*.h declares.

No compute call is made here (this container has no GPU)."""
import ctypes
import glob
import os
import re

import pytest

from vdn_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for path in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\**\s*(vdn_[a-z0-9_]+)\s*\(", text, re.M)
    return sorted(set(names))


def test_header_declares_the_bound_signatures():
    declared = declared_functions()
    assert declared, "no declarations parsed from include/*.h"
    assert sorted(_lib.exported_symbols()) == declared


def test_library_loads_and_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIBRARY_PATH):
        pytest.fail("libvdnmi.so is not built; run __graft_entry__.build()")
    lib = _lib.load()
    for name in declared_functions():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name
    assert lib.vdn_abi_version() == 6
    assert lib.vdn_last_error() is not None


def test_invalid_arguments_are_rejected_without_a_device():
    lib = _lib.load()
    # Argument validation happens before any HIP call, so these run on a CPU-only host.
    assert lib.vdn_mxfp8_quantize(None, 4, 0, 4, None, None, None, None) != 0
    assert b"K > 0" in lib.vdn_last_error()
    assert lib.vdn_mxfp8_gemm(None, None, 128, None, None, 128, 128, None, None, 0, None, 0,
                              None, None, 1, 1, 1, None, None) != 0
    assert b"null pointer" in lib.vdn_last_error()


def test_short_conv_and_swiglu_entry_points_validate_before_launching():
    """The fused short-conv prepare and the SwiGLU producer reject bad arguments before any
    HIP call (fake, never dereferenced, 256-aligned addresses)."""
    lib = _lib.load()
    fake = 1 << 20
    assert lib.vdn_vda_conv_prepare(None, 2, 256, 128, 3, 4, 5, fake, fake, 1, fake, None) != 0
    assert b"null pointer" in lib.vdn_last_error()
    assert lib.vdn_vda_conv_prepare(fake, 2, 256, 128, 3, 0, 5, fake, fake, 1, fake, None) != 0
    assert b"positive" in lib.vdn_last_error()
    assert lib.vdn_vda_conv_prepare(fake, 2, 250, 128, 3, 4, 5, fake, fake, 1, fake, None) != 0
    assert b"16-byte" in lib.vdn_last_error()
    # heads that do not fit inside a row
    assert lib.vdn_vda_conv_prepare(fake, 3, 256, 128, 3, 4, 5, fake, fake, 1, fake, None) != 0
    assert b"inside a row" in lib.vdn_last_error()
    # SwiGLU needs the interleaved weight: padded N = 2 pad128(n)
    assert lib.vdn_mxfp8_gemm_act_quantize(fake, fake, 2048, fake, fake, 1280, 256, None, 2, fake,
                                           fake, 2048, 700, None, None) != 0
    assert b"interleaved" in lib.vdn_last_error()
    assert lib.vdn_mxfp8_gemm_act_quantize(fake, fake, 2048, fake, fake, 1280, 256, None, 3, fake,
                                           fake, 2048, 640, None, None) != 0
    assert b"unknown activation" in lib.vdn_last_error()


def test_vda_readout_and_epilogue_validate_head_dim():
    """head_dim (ABI 4) must be 16, 32, 64 or 128; checked before any HIP call (fake, never
    dereferenced, aligned addresses)."""
    lib = _lib.load()
    fake = 1 << 20
    args = (fake, 1024, 512, 128, 1, fake, fake, 0, 1e-6, fake, 1024, 512, 128, fake, 1024, 128,
            512)
    assert lib.vdn_vda_readout(*args, 48, 2, 4, 8, None) != 0
    assert b"head_dim" in lib.vdn_last_error()
    assert lib.vdn_vda_epilogue(fake, fake, 0, 1e-6, fake, 1024, 512, 128, fake, 1024, 128, 512,
                                256, 2, 4, 8, None) != 0
    assert b"head_dim" in lib.vdn_last_error()
