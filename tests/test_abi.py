"""The C-ABI library loads and exports every symbol include/z2h.h declares (no device calls)."""
import ctypes as C
import re

from zonos2_amd.lib import BUILD


def test_exports_match_header(root):
    hdr = (root / "include" / "z2h.h").read_text()
    decl = set(re.findall(r"\b(z2h_[a-z_]+)\s*\(", hdr))
    assert len(decl) >= 15
    lib = C.CDLL(str(BUILD / "libzonos2_hip.so"))
    missing = [n for n in sorted(decl) if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header(root):
    from zonos2_amd import z2h
    hdr = (root / "include" / "z2h.h").read_text()
    decl = set(re.findall(r"\b(z2h_[a-z_]+)\s*\(", hdr))
    assert decl == set(z2h.EXPORTS)
