"""In-tree build of the gfx950 engine library and its PyTorch-ROCm extension.

    python -m cugo_amd.build          (or __graft_entry__.build())

Produces, next to this file:
  libcugo_hip.so            kernels + C ABI (include/cugo_hip.h), hipcc --offload-arch=gfx950
  cugo_torch50_ext*.so      pybind module mirroring the reference extension's operations
and the generated csrc/stop_bits.inc table (the host C library's log2f, see below).
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
import sysconfig
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
ARCH = os.environ.get("CUGO_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Shared by every HIP compile: IEEE fp32 division, no contraction, no packed fp32.  The
# packed-fp32 feature switch applies to the device pass (a float2 multiply-add probe
# compiles to one packed FMA without it and to two scalar ones with it); hipcc's host pass
# warns that it does not know the feature.  check_no_packed_fp32() verifies the result.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

EXT_NAME = "_cugo_torch50_hip"


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True, cwd=cwd)


def _newer(target: Path, sources: list[Path]) -> bool:
    return target.exists() and all(target.stat().st_mtime >= s.stat().st_mtime for s in sources)


def generate_stop_bits(force: bool = True) -> Path:
    """Writes csrc/stop_bits.inc: log2f(1 + p) / 12, clamped to 1, for p in [0, 4095).

    The reference encoder evaluates this with the C library's log2f at run time
    (include/cugo/game/torch50.h:405-408).  Evaluating the same call on the build host
    and baking the 4,095 floats into the kernel keeps the feature bit-exact without
    reimplementing log2f on the GPU."""
    out = CSRC / "stop_bits.inc"
    gen_src = CSRC / "gen_stop_bits.c"
    gen_bin = PKG / "_gen_stop_bits"
    if not force and _newer(out, [gen_src]):
        return out
    _run(["gcc", "-O0", "-std=c11", "-fno-fast-math", "-ffp-contract=off", str(gen_src),
          "-o", str(gen_bin), "-lm"])
    text = subprocess.run([str(gen_bin)], check=True, capture_output=True, text=True).stdout
    out.write_text(text)
    gen_bin.unlink(missing_ok=True)
    return out


LLVM_BIN = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "llvm" / "bin"
PACKED_FP32 = re.compile(r"\bv_pk_(add|mul|fma)_f32\b")
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def device_disassembly(lib: Path) -> str:
    """The gfx950 disassembly of every code object in `lib`'s .hip_fatbin section (one
    offload bundle per source file, concatenated)."""
    with tempfile.TemporaryDirectory() as tmp:
        fatbin = Path(tmp) / "fatbin"
        _run(["objcopy", "--dump-section", f".hip_fatbin={fatbin}", str(lib)])
        data = fatbin.read_bytes()
        starts = [m.start() for m in re.finditer(re.escape(BUNDLE_MAGIC), data)]
        text = []
        for k, begin in enumerate(starts):
            end = starts[k + 1] if k + 1 < len(starts) else len(data)
            part, obj = Path(tmp) / f"b{k}", Path(tmp) / f"b{k}.co"
            part.write_bytes(data[begin:end])
            _run([str(LLVM_BIN / "clang-offload-bundler"), "--type=o",
                  f"--targets=hipv4-amdgcn-amd-amdhsa--{ARCH}", f"--input={part}",
                  f"--output={obj}", "--unbundle"])
            text.append(subprocess.run([str(LLVM_BIN / "llvm-objdump"), "-d", str(obj)],
                                       check=True, capture_output=True, text=True).stdout)
        return "\n".join(text)


def check_no_packed_fp32(lib: Path) -> None:
    """Fails the build when the device code holds a packed fp32 add, multiply or FMA (some
    of their forms have given wrong results on this hardware without an error)."""
    asm = device_disassembly(lib)
    if not asm.strip():
        raise RuntimeError(f"{lib}: no device code found to check")
    hits = sorted({m.group(0) for m in PACKED_FP32.finditer(asm)})
    if hits:
        raise RuntimeError(f"{lib}: packed fp32 instructions in device code: {hits}")
    print(f"  {lib.name}: no packed fp32 instructions in {asm.count(chr(10))} lines of "
          "device code", flush=True)


SOURCES = ("kernels.hip", "decode.hip", "selfplay.hip", "mlp.hip", "linear.hip")
HEADERS = (CSRC / "engine.h", REPO / "include" / "cugo_hip.h")


def build_library(force: bool = True) -> Path:
    """Compiles each source to an object under _build/ (in parallel; with force=False only
    those older than their source or a shared header), then links the library."""
    generate_stop_bits(force=force)
    out = PKG / "libcugo_hip.so"
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    shared = [*HEADERS, CSRC / "stop_bits.inc"]
    procs, objs = [], []
    for name in SOURCES:
        src, obj = CSRC / name, objdir / (name + ".o")
        objs.append(obj)
        if force or not _newer(obj, [src, *shared]):
            cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
            print("+", " ".join(cmd), flush=True)
            procs.append((name, subprocess.Popen(cmd)))
    failed = [name for name, p in procs if p.wait() != 0]
    if failed:
        raise RuntimeError(f"hipcc failed for {failed}")
    if procs or not _newer(out, objs):
        _run([HIPCC, *HIP_FLAGS, "-shared", *map(str, objs), "-o", str(out)])
        check_no_packed_fp32(out)
    return out


def _ext_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def build_extension() -> Path:
    import torch
    from torch.utils import cpp_extension

    out = PKG / f"{EXT_NAME}{_ext_suffix()}"
    includes = cpp_extension.include_paths(device_type="cuda")
    libdirs = cpp_extension.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{p}" for p in includes],
        f"-I{sysconfig.get_paths()['include']}",
        str(CSRC / "torch_ext.cpp"),
        "-o", str(out),
        f"-L{PKG}", "-lcugo_hip",
        *[f"-L{p}" for p in libdirs],
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
        "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
    ]
    _run(cmd)
    return out


def build_oracle() -> None:
    """The oracle's C restatement always; oracle/_ref from the reference checkout when it
    is present (test infrastructure, never loaded by the package)."""
    targets = ["oracle"]
    if Path(os.environ.get("CUGO_REFERENCE_INCLUDE", "/root/reference/include")).is_dir():
        targets.append("ref")
    _run(["make", "-s", "-C", str(REPO / "oracle"), *targets])


def build_all() -> None:
    build_library()
    build_extension()
    build_oracle()


if __name__ == "__main__":
    what = sys.argv[1:] or ["all"]
    for item in what:
        {"all": build_all, "lib": build_library, "ext": build_extension,
         "oracle": build_oracle, "lib-changed": lambda: build_library(force=False)}[item]()
