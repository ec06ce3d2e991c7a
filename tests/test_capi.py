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


def test_route_query_and_environment(monkeypatch):
    lib = _lib.load()
    monkeypatch.delenv("CVN_DISABLE_FUSED", raising=False)
    assert lib.cvn_converse2d_route(16, 64, 256, 256, 1, 5, 5, 1, 2) == _lib.ROUTE_FUSED  # 260^2
    assert lib.cvn_converse2d_route(8, 128, 256, 256, 1, 7, 7, 1, 6) == _lib.ROUTE_PFA268  # 268^2
    assert lib.cvn_converse2d_route(8, 64, 64, 64, 1, 3, 3, 2, 1) == _lib.ROUTE_FUSED  # cfg2: 66 -> 132
    assert lib.cvn_converse2d_route(8, 64, 60, 60, 1, 3, 3, 2, 1) == _lib.ROUTE_GENERIC  # 62 -> 124
    assert lib.cvn_converse2d_route(16, 64, 260, 260, 1, 5, 5, 1, 0) == _lib.ROUTE_FUSED  # padded input, op path
    assert lib.cvn_converse2d_route(16, 64, 258, 258, 1, 5, 5, 1, 1) == _lib.ROUTE_GENERIC  # 258 % 4 != 0
    # 256^2 planes (Converse-USRNet's data steps, per-sample 25 x 25 psf): the Cooley-Tukey fused plan
    assert lib.cvn_converse2d_route(4, 64, 256, 256, 4, 25, 25, 1, 0) == _lib.ROUTE_FUSED
    assert lib.cvn_converse2d_route(1, 2, 240, 240, 1, 7, 7, 1, 8) == _lib.ROUTE_FUSED
    assert lib.cvn_converse2d_route(1, 2, 250, 250, 1, 7, 7, 1, 3) == _lib.ROUTE_GENERIC  # 250 % 4 != 0
    assert lib.cvn_converse2d_route(4, 64, 64, 64, 4, 25, 25, 4, 0) == _lib.ROUTE_FUSED  # 64 -> 256 up plan
    assert lib.cvn_converse2d_route(4, 64, 128, 128, 4, 25, 25, 2, 0) == _lib.ROUTE_GENERIC  # 128 -> 256: no up plan
    monkeypatch.setenv("CVN_DISABLE_FUSED", "1")
    assert lib.cvn_converse2d_route(16, 64, 256, 256, 1, 5, 5, 1, 2) == _lib.ROUTE_GENERIC
    assert lib.cvn_converse2d_route(8, 128, 256, 256, 1, 7, 7, 1, 6) == _lib.ROUTE_GENERIC
    # an explicit route does not read the environment: the fused table size is still available
    assert lib.cvn_converse2d_table_bytes(16, 64, 256, 256, 1, 5, 5, 1, 2, _lib.ROUTE_FUSED) > 0
    assert lib.cvn_converse2d_route(1, 3, 5000, 8, 1, 3, 3, 1, 1) == _lib.CVN_ERR_UNSUPPORTED


def test_explicit_route_must_serve_geometry_and_table_size_is_checked():
    lib = _lib.load()
    geo = (8, 64, 60, 60, 1, 3, 3, 2, 1)  # s = 2 onto a 124 x 124 plane: only the generic route serves it
    assert lib.cvn_converse2d_table_bytes(*geo, _lib.ROUTE_FUSED) == 0
    assert lib.cvn_converse2d_table_bytes(*geo, _lib.ROUTE_PFA268) == 0
    assert lib.cvn_converse2d_table_bytes(*geo, 7) == 0
    tb = lib.cvn_converse2d_table_bytes(*geo, _lib.ROUTE_GENERIC)
    sb = lib.cvn_converse2d_scratch_bytes(*geo, _lib.ROUTE_GENERIC)
    assert tb > 0 and sb > 0
    assert lib.cvn_converse2d_fwd_workspace(*geo) >= tb + sb
    B, C, H, W, pb, kh, kw, s, p = geo
    dummy = 256  # never dereferenced: argument checks fail first
    rc = lib.cvn_converse2d_apply_f32(dummy, B, C, H, W, pb, kh, kw, s, p, 3, 0, _lib.ROUTE_FUSED, dummy, tb, dummy,
                                      sb, dummy, None)
    assert rc == _lib.CVN_ERR_ARG and b"route" in lib.cvn_last_error()
    rc = lib.cvn_converse2d_apply_f32(dummy, B, C, H, W, pb, kh, kw, s, p, 3, 0, _lib.ROUTE_GENERIC, dummy, tb - 1,
                                      dummy, sb, dummy, None)
    assert rc == _lib.CVN_ERR_ARG and b"table" in lib.cvn_last_error()
    # the fused route asks for scratch only where it splits planes over two workgroups (<= 128 planes)
    assert lib.cvn_converse2d_scratch_bytes(1, 64, 128, 128, 1, 5, 5, 1, 2, _lib.ROUTE_FUSED) > 0
    assert lib.cvn_converse2d_scratch_bytes(2, 64, 128, 128, 1, 5, 5, 1, 2, _lib.ROUTE_FUSED) > 0
    assert lib.cvn_converse2d_scratch_bytes(3, 43, 128, 128, 1, 5, 5, 1, 2, _lib.ROUTE_FUSED) == 0
    assert lib.cvn_converse2d_scratch_bytes(16, 64, 256, 256, 1, 5, 5, 1, 2, _lib.ROUTE_FUSED) == 0
    assert lib.cvn_converse2d_scratch_bytes(8, 64, 64, 64, 1, 3, 3, 2, 1, _lib.ROUTE_FUSED) == 0  # scale 2
    g1 = (1, 64, 128, 128, 1, 5, 5, 1, 2)
    assert lib.cvn_converse2d_fwd_workspace(*g1) >= (lib.cvn_converse2d_table_bytes(*g1, _lib.ROUTE_FUSED)
                                                     + lib.cvn_converse2d_scratch_bytes(*g1, _lib.ROUTE_FUSED))
    # the fused (260^2) and 268 tables differ from the generic table of the same geometry
    g260 = (16, 64, 256, 256, 1, 5, 5, 1, 2)
    assert lib.cvn_converse2d_table_bytes(*g260, _lib.ROUTE_FUSED) != lib.cvn_converse2d_table_bytes(
        *g260, _lib.ROUTE_GENERIC)


def test_support_query_matches_library_limits():
    lib = _lib.load()
    ok = lambda *a: lib.cvn_converse2d_supported(*a) == _lib.CVN_OK  # noqa: E731
    assert ok(16, 64, 256, 256, 1, 5, 5, 1, 2, 0, 0)
    assert ok(16, 64, 256, 256, 1, 5, 5, 1, 2, 1, 1)
    assert not ok(1, 3, 5000, 8, 1, 3, 3, 1, 1, 0, 0)          # padded side above 4096
    assert lib.cvn_converse2d_supported(1, 3, 5000, 8, 1, 3, 3, 1, 1, 0, 0) == _lib.CVN_ERR_UNSUPPORTED
    assert not ok(300, 300, 32, 32, 1, 3, 3, 2, 1, 0, 0)       # generic path: B*C above 65535
    assert ok(300, 300, 128, 128, 1, 5, 5, 1, 2, 0, 0)         # fused path: no such limit
    assert not ok(300, 300, 128, 128, 1, 5, 5, 1, 2, 1, 0)     # ... but the backward has it
    assert not ok(1, 2, 8, 8, 1, 3, 3, 5, 1, 0, 1)             # weight gradients: scale <= 4
    assert ok(1, 2, 8, 8, 1, 3, 3, 5, 1, 1, 0)                 # grad_x alone: any scale
    assert not ok(1, 1, 2200, 2200, 1, 3, 3, 1, 1, 0, 1)       # weight-gradient tables above 64 KiB
    assert ok(1, 1, 2100, 2100, 1, 3, 3, 1, 1, 1, 0)           # grad_x at a 2100 side
    assert not ok(1, 1, 3000, 3000, 1, 3, 3, 1, 1, 1, 0)       # backward column pass above 160 KiB
    assert not ok(2, 3, 8, 8, 3, 3, 3, 1, 1, 0, 0)             # psf batch neither 1 nor B


def test_op_split_sizes_add_up():
    lib = _lib.load()
    for (B, C, h, w, k, s) in [(2, 3, 20, 18, 3, 1), (8, 64, 66, 66, 3, 2), (1, 4, 30, 26, 25, 4)]:
        tb = lib.cvn_converse2d_op_table_bytes(C, h, w, k, k, s)
        sb = lib.cvn_converse2d_op_scratch_bytes(B, C, h, w, s)
        assert tb > 0 and sb > 0
        assert lib.cvn_converse2d_op_workspace(B, C, h, w, k, k, s) == tb + sb
        # the op table does not depend on the batch
        assert lib.cvn_converse2d_op_table_bytes(C, h, w, k, k, s) == tb
    assert lib.cvn_converse2d_op_table_bytes(3, 5000, 8, 3, 3, 1) == 0


def test_op_route_query():
    """The op path runs the compile-time-plan kernels exactly for scale 2-4, h in {64, 128, 256} and w,
    w * scale in the planned lengths; everything else (scale 1 included) takes the generic kernels."""
    lib = _lib.load()
    planned, generic = _lib.ROUTE_OP_PLANNED, _lib.ROUTE_GENERIC
    for h, w, s in [(256, 256, 2), (256, 256, 3), (256, 256, 4), (64, 64, 2), (128, 64, 3), (64, 256, 4),
                    (256, 128, 3), (128, 192, 2), (64, 64, 3), (128, 128, 2)]:
        assert lib.cvn_converse2d_op_route(h, w, s) == planned, (h, w, s)
    for h, w, s in [(256, 256, 1), (256, 256, 5), (260, 256, 2), (256, 260, 2), (32, 64, 2), (256, 40, 2),
                    (96, 96, 2), (20, 22, 3), (0, 64, 2), (5000, 64, 2)]:
        assert lib.cvn_converse2d_op_route(h, w, s) == generic, (h, w, s)


def test_noalloc_limit_and_rejection_without_device():
    lib = _lib.load()
    text = open(HEADER).read()
    m = re.search(r"#define CVN_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES
    # above the array's size: rejected before any device call
    rc = lib.cvn_converse2d_fwd_noalloc_f32(256, 8, 128, 256, 256, 256, 1, 7, 7, 256, 1e-5, 1, 6, 3, 0, 256, None)
    assert rc == _lib.CVN_ERR_UNSUPPORTED and b"scratch" in lib.cvn_last_error()
    # invalid geometry: the forward's own argument error
    rc = lib.cvn_converse2d_fwd_noalloc_f32(None, 1, 2, 8, 8, None, 3, 3, 3, None, 1e-5, 1, 1, 3, 0, None, None)
    assert rc == _lib.CVN_ERR_ARG
