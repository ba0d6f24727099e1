"""The C++ boundary a reference caller compiles against (include/zonos2.h + include/zonos2-sampler.h).

- A caller shaped like the reference server's decode worker (tests/native/server_surface.cpp: the
  server's zonos2_* calls, batch-context fields, hparams, prompt options and the backend name that
  replaces ggml_backend_name(model.backend)) compiles against the header.
- The reference's own prompt builder, src/zonos2-prompt.cpp, compiles unchanged against this header
  (it reads only model.hp) when the reference tree is present, and the caller then links against
  libzonos2.so plus that object with no duplicate or missing symbol: the link recipe of
  INTEGRATION.md, minus the reference's static zonos2 library.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BUILD = ROOT / "zonos2.cpp_amd" / "build"
REF_PROMPT = Path("/root/reference/src/zonos2-prompt.cpp")
FLAGS = ["-std=c++17", "-O0", f"-I{ROOT / 'include'}"]


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, capture_output=True, text=True, cwd=cwd)
    assert r.returncode == 0, r.stdout + r.stderr
    return r


def test_server_shaped_caller_compiles(tmp_path):
    _run(["g++", *FLAGS, "-c", str(ROOT / "tests" / "native" / "server_surface.cpp"), "-o", str(tmp_path / "s.o")])


@pytest.mark.skipif(not REF_PROMPT.exists(), reason="the reference tree is not on this machine")
def test_reference_prompt_builder_compiles_and_links_against_the_library(tmp_path):
    if not (BUILD / "libzonos2.so").exists():
        pytest.skip("libzonos2.so not built")
    # the reference's file unchanged, against this header: fed on stdin from another directory, so its
    # #include "zonos2.h" cannot pick up the ggml header beside it (a maintainer's build compiles a
    # staged copy in its build directory for the same reason)
    with open(REF_PROMPT) as src:
        r = subprocess.run(["g++", *FLAGS, "-x", "c++", "-c", "-", "-o", str(tmp_path / "prompt.o")], stdin=src,
                           capture_output=True, text=True, cwd=tmp_path)
    assert r.returncode == 0, r.stdout + r.stderr
    _run(["g++", *FLAGS, "-c", str(ROOT / "tests" / "native" / "server_surface.cpp"), "-o", str(tmp_path / "s.o")])
    _run(["g++", str(tmp_path / "s.o"), str(tmp_path / "prompt.o"), "-o", str(tmp_path / "server_surface"),
          f"-L{BUILD}", "-lzonos2", "-lzonos2_hip", f"-Wl,-rpath,{BUILD}", "-Wl,--no-undefined",
          "-Wl,--unresolved-symbols=ignore-in-shared-libs"])
    assert (tmp_path / "server_surface").exists()
