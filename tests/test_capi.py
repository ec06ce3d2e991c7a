"""The C-ABI library loads without a GPU, exports every symbol include/converse2d.h declares, and
rejects bad arguments before touching the device."""
import ctypes
import os
import re

import pytest

from conversenet_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "converse2d.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cvn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "cvn_converse2d_fwd_f32" in names and "cvn_converse2d_op_f32" in names
    assert len(names) >= 12


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    assert sorted(_lib.SIGNATURES) == declared()


def test_version_and_error_string():
    lib = _lib.load()
    assert b"gfx950" in lib.cvn_version()
    assert lib.cvn_clear_cache() == 0


def test_argument_errors_without_device():
    lib = _lib.load()
    # workspace query returns 0 for invalid shapes
    assert lib.cvn_converse2d_fwd_workspace(1, 0, 8, 8, 1, 3, 3, 1, 1) == 0
    assert lib.cvn_converse2d_fwd_workspace(2, 3, 8, 8, 3, 3, 3, 1, 1) == 0  # psf batch neither 1 nor B
    assert lib.cvn_converse2d_fwd_workspace(1, 3, 8, 8, 1, 3, 3, 0, 1) == 0  # scale 0
    assert lib.cvn_converse2d_fwd_workspace(1, 3, 8, 8, 1, 3, 3, 1, 1) > 0
    # null pointers / bad modes fail with CVN_ERR_ARG and a message
    rc = lib.cvn_converse2d_fwd_f32(None, 1, 2, 8, 8, None, 1, 3, 3, None, 1e-5, 1, 1, 3, 0, None, None, 0, None)
    assert rc == _lib.CVN_ERR_ARG and b"null" in lib.cvn_last_error()
    rc = lib.cvn_converse2d_fwd_f32(None, 1, 2, 8, 8, None, 1, 3, 3, None, 1e-5, 1, 1, 9, 0, None, None, 0, None)
    assert rc == _lib.CVN_ERR_ARG and b"padding mode" in lib.cvn_last_error()
    rc = lib.cvn_converse2d_fwd_f32(None, 1, 2, 8, 8, None, 1, 3, 3, None, 1e-5, 1, 8, 1, 0, None, None, 0, None)
    assert rc == _lib.CVN_ERR_ARG and b"reflect" in lib.cvn_last_error()
    big = lib.cvn_converse2d_fwd_f32(None, 1, 1, 5000, 8, None, 1, 3, 3, None, 1e-5, 1, 1, 3, 0, None, None, 0, None)
    assert big == _lib.CVN_ERR_UNSUPPORTED
    assert lib.cvn_layernorm_cf_f32(None, 1, 2, 4, None, None, 1e-6, None, None) == _lib.CVN_ERR_ARG
    assert lib.cvn_conv1x1_f32(None, 1, 2, 4, None, None, 2, 0, None, None, None, None) == _lib.CVN_ERR_ARG
    assert lib.cvn_copy_f32(None, None, 4, None) == _lib.CVN_ERR_ARG


def test_fwd_workspace_accounts_for_scale():
    lib = _lib.load()
    w1 = lib.cvn_converse2d_fwd_workspace(2, 4, 16, 16, 1, 3, 3, 1, 1)
    w2 = lib.cvn_converse2d_fwd_workspace(2, 4, 16, 16, 1, 3, 3, 2, 1)
    assert w2 > 3 * w1
