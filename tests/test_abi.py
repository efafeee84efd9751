"""The C ABI library loads, exports every entry point include/mira_rocm.h declares,
and its struct layouts match the ctypes binding (no GPU needed)."""
import ctypes as C
import os
import re

from mira_amd import _lib as L

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "mira_rocm.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mr_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_exports():
    assert declared_functions() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_struct_sizes():
    lib = L.load()
    assert lib.mr_abi_version() == L.ABI_VERSION
    assert lib.mr_sizeof(b"mr_epi_step") == C.sizeof(L.EpiStep) == 32
    assert lib.mr_sizeof(b"mr_epilogue") == C.sizeof(L.Epilogue)
    assert lib.mr_sizeof(b"mr_conv_geom") == C.sizeof(L.ConvGeom) == 64
    assert lib.mr_sizeof(b"nope") == -1


def test_invalid_arguments_are_rejected_before_any_launch():
    """Host-side validation returns MR_EINVAL with a message; no device call is made."""
    lib = L.load()
    e = L.Epilogue()
    assert lib.mr_qmatmul(None, 16, None, 64, 32, 4, 8, 16, C.byref(e), None) == 1
    assert b"NULL" in lib.mr_last_error()
    assert lib.mr_quantize_rows(None, 1, 1, 1, None, 4, 1.0, None) == 1
    g = L.ConvGeom(n=1, h=8, w=8, c=3, c_pad=8, o=4, oh=8, ow=8, kh=3, kw=3, sh=1, sw=1, ph=1, pw=1, dh=1, dw=1)
    assert lib.mr_qconv2d(C.c_void_p(16), C.byref(g), C.c_void_p(16), 64, 32, C.byref(e), None) == 1
    assert b"c_pad" in lib.mr_last_error()


def test_fused_stem_declines_what_it_cannot_fuse():
    """mr_qconv2d_maxpool answers MR_EUNSUPPORTED (3) for pool shapes without a kernel and
    for epilogues the pool does not commute with (a mul is accepted only per channel or
    scalar: the caller guarantees its operand positive); the caller then runs conv and pool
    apart."""
    lib = L.load()
    g = L.ConvGeom(n=1, h=224, w=224, c=3, c_pad=4, o=64, oh=112, ow=112, kh=7, kw=7, sh=2, sw=2, ph=3, pw=3,
                   dh=1, dw=1)
    x, b = C.c_void_p(256), C.c_void_p(256)
    e = L.Epilogue()
    e.n_steps = 2
    e.steps[0].fn, e.steps[0].mode = L.EPI_FN["add"], L.BC_COL
    e.steps[1].fn = L.EPI_FN["relu"]
    inf = float("-inf")
    assert lib.mr_qconv2d_maxpool(x, C.byref(g), b, 256, 64, C.byref(e), 3, 3, 1, 1, inf, 38, 38, None) == 3
    assert b"no kernel" in lib.mr_last_error()
    for fn, mode, swapped in (("mul", L.BC_ROW, 0), ("add", L.BC_FULL, 0), ("add", L.BC_ROW, 0),
                              ("sub", L.BC_SCALAR, 1), ("div", L.BC_SCALAR, 0)):
        e.steps[0].fn, e.steps[0].mode, e.steps[0].swapped = L.EPI_FN[fn], mode, swapped
        assert lib.mr_qconv2d_maxpool(x, C.byref(g), b, 256, 64, C.byref(e), 3, 2, 1, 1, inf, 56, 56, None) == 3
        assert b"non-decreasing" in lib.mr_last_error()
