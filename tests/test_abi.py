"""CPU checks of the drop-in boundary: the library loads and exports what include/anima.h
declares, and host-side validation fails cleanly without a device."""

import ctypes

import pytest

from helpers import amd


def test_header_declares_entry_points():
    syms = amd().declared_symbols()
    for s in ("anima_init", "anima_attention", "anima_qk_norm_rope", "anima_rmsnorm", "anima_rope",
              "anima_alloc", "anima_free", "anima_h2d", "anima_d2h", "anima_sync", "anima_last_error"):
        assert s in syms, s


def test_library_exports_every_declared_symbol():
    lib = amd().lib()
    missing = [s for s in amd().declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_init_without_device_reports_error():
    # no GPU in this container: anima_init must fail with a status and a message, not crash
    m = amd()
    h = ctypes.c_void_p()
    rc = m.lib().anima_init(0, ctypes.byref(h))
    if rc == 0:
        m.lib().anima_destroy(h)
        pytest.skip("a GPU is visible; covered by the gpu tests")
    assert rc < 0
    assert m.lib().anima_last_error(None)


def test_null_context_is_rejected():
    m = amd()
    assert m.lib().anima_sync(None) == -1
    assert m.lib().anima_attention(None, None) == -1


def test_binding_struct_layouts_match_the_library():
    """Every descriptor struct the ctypes binding restates has the library's size and field
    offsets (anima_abi_offset); a planted layout change is detected."""
    m = amd()
    assert m.abi_mismatches(m.lib()) == []
    L = m.lib()
    assert L.anima_abi_offset(b"anima_attn_desc", b"no_such_field") == -1
    assert L.anima_abi_offset(b"no_such_struct", None) == -1

    class Shifted(ctypes.Structure):  # kv_prep_bytes dropped: the size differs
        _fields_ = m.AttnDesc._fields_[:-1]

    saved = m.ABI_STRUCTS["anima_attn_desc"]
    m.ABI_STRUCTS["anima_attn_desc"] = Shifted
    try:
        assert any("sizeof(anima_attn_desc)" in b for b in m.abi_mismatches(L))
    finally:
        m.ABI_STRUCTS["anima_attn_desc"] = saved
