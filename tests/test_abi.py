"""The C-ABI library loads and exports every symbol include/z2h.h declares (no device calls)."""
import ctypes as C
import re

from zonos2_amd.lib import BUILD

# function declarations only: a return type at the start of a line, then the z2h_ name and "("
DECL = re.compile(r"^(?:int|int64_t|void|const char \*)\s+\**\s*(z2h_[a-z0-9_]+)\s*\(", re.M)


def test_exports_match_header(root):
    hdr = (root / "include" / "z2h.h").read_text()
    decl = set(DECL.findall(hdr))
    assert len(decl) >= 15
    lib = C.CDLL(str(BUILD / "libzonos2_hip.so"))
    missing = [n for n in sorted(decl) if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header(root):
    from zonos2_amd import z2h
    hdr = (root / "include" / "z2h.h").read_text()
    decl = set(DECL.findall(hdr))
    assert decl == set(z2h.EXPORTS)


def test_cpp_api_library_defines_the_header_functions(root):
    """libzonos2.so defines every function include/zonos2.h declares, zonos2_generate included,
    except zonos2_build_prompt (compiled from the reference's own src/zonos2-prompt.cpp)."""
    import subprocess
    hdr = (root / "include" / "zonos2.h").read_text()
    names = set(re.findall(r"^[A-Za-z_][\w:<>\s\*&]*?\b(zonos2_[a-z0-9_]+)\s*\(", hdr, re.M)) - {"zonos2_build_prompt"}
    assert {"zonos2_generate", "zonos2_batch_step", "zonos2_batch_slot_prefill"} <= names
    out = subprocess.run(["nm", "-D", "-C", "--defined-only", str(BUILD / "libzonos2.so")], capture_output=True,
                         text=True, check=True).stdout
    missing = [n for n in sorted(names) if f" {n}(" not in out]
    assert not missing, missing
