"""Build the native libraries in-tree (no JIT caches, so the built .so files travel with the tree).

  build/libzonos2_host.so : host C++ (synthetic weights, GGUF-format quantizers, GGUF I/O)
  build/libzonos2_hip.so  : the gfx950 HIP kernels behind the C ABI of include/z2h.h
  build/libzonos2.so      : the ggml-free zonos2.h batch API (C++), layered on libzonos2_hip.so
  build/zonos2-batch      : CLI with the reference's --batch-test / --decode-bench semantics
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
BUILD = PKG / "build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: no packed fp32 math (v_pk_*_f32); some of its forms have returned wrong results
# on this hardware without any error, so every kernel is built with it off.
HIP_FLAGS = [
    "-O3", f"--offload-arch={ARCH}", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
]
HOST_FLAGS = ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fPIC", "-std=c++17", "-pthread", "-Wall"]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


def _stale(out: Path, deps: list[Path]) -> bool:
    if not out.exists():
        return True
    t = out.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def build_host(force: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    out = BUILD / "libzonos2_host.so"
    srcs = [PKG / "host" / "z2_synth.cpp", PKG / "host" / "gguf.cpp"]
    deps = srcs + [PKG / "host" / "z2_formats.h", PKG / "host" / "gguf.h"]
    if force or _stale(out, deps):
        _run(["g++", *HOST_FLAGS, "-shared", *map(str, srcs), "-o", str(out)])
    return out


def build_hip(force: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    out = BUILD / "libzonos2_hip.so"
    csrc = PKG / "csrc"
    srcs = [csrc / "z2h.hip", csrc / "z2h_tp.hip"]
    deps = srcs + sorted(csrc.glob("*.h")) + [ROOT / "include" / "z2h.h", PKG / "host" / "z2_formats.h"]
    if force or _stale(out, deps):
        _run([HIPCC, *HIP_FLAGS, "-shared", f"-I{ROOT / 'include'}", f"-I{PKG / 'host'}",
              *map(str, srcs), "-o", str(out)])
    return out


def build_api(force: bool = True) -> tuple[Path, Path]:
    """zonos2.h C++ API over the C ABI, plus the batch-test / decode-bench CLI."""
    BUILD.mkdir(exist_ok=True)
    lib = BUILD / "libzonos2.so"
    cli = BUILD / "zonos2-batch"
    host = PKG / "host"
    srcs = [host / "zonos2_batch.cpp", host / "gguf.cpp", host / "zonos2_sampler.cpp", host / "zonos2_generate.cpp"]
    deps = srcs + [ROOT / "include" / "zonos2.h", ROOT / "include" / "zonos2-sampler.h", ROOT / "include" / "z2h.h", host / "gguf.h"]
    inc = [f"-I{ROOT / 'include'}", f"-I{host}"]
    rpath = "-Wl,-rpath,$ORIGIN"
    if force or _stale(lib, deps):
        _run(["g++", *HOST_FLAGS, *inc, "-shared", *map(str, srcs), "-o", str(lib),
              f"-L{BUILD}", "-lzonos2_hip", rpath])
    cli_src = host / "zonos2_batch_cli.cpp"
    if force or _stale(cli, [cli_src, lib]):
        _run(["g++", *HOST_FLAGS, *inc, str(cli_src), "-o", str(cli), f"-L{BUILD}", "-lzonos2",
              "-lzonos2_hip", "-lzonos2_host", rpath])
    # the generation known-answer program the GPU tests run (tests/native/generate_kat.cpp)
    kat_src = ROOT / "tests" / "native" / "generate_kat.cpp"
    kat = BUILD / "generate_kat"
    if kat_src.exists() and (force or _stale(kat, [kat_src, lib])):
        _run(["g++", *HOST_FLAGS, *inc, str(kat_src), "-o", str(kat), f"-L{BUILD}", "-lzonos2", "-lzonos2_hip", rpath])
    return lib, cli


def build_oracle(force: bool = True) -> Path:
    args = ["make", "-C", str(ROOT / "oracle"), "-j4"]
    if force:
        _run(["make", "-C", str(ROOT / "oracle"), "clean"])
    _run(args)
    return ROOT / "oracle" / "build" / "liboracle.so"


def build_all(force: bool = True, api: bool = True) -> None:
    build_host(force)
    build_hip(force)
    if api and (PKG / "host" / "zonos2_batch.cpp").exists():
        build_api(force)
    build_oracle(force)


if __name__ == "__main__":
    build_all(force="--force" in sys.argv or True)
    print("built:", *sorted(p.name for p in BUILD.iterdir()))
