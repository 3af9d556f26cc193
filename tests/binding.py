"""Builds the compiled C/C++ consumers of include/slime_ca.h (test programs).

* ``compile_header(lang)``: a translation unit holding only ``#include
  "slime_ca.h"``, compiled as C99 (gcc) or C++17 (g++) with -Wall -Wextra -Werror
  -pedantic: the header stands on its own for a C or C++ host.
* ``build_binding()``: ``tests/ca_binding.cpp`` (the reference-side binding of the
  library, as a C++ host program) compiled with g++ and linked against
  ``slime_amd/libslime_ca.so`` and the HIP runtime, into ``tests/_build/ca_binding``
  with an rpath to the library, so the binary runs from any working directory and
  travels with the tree.

``__graft_entry__.build()`` calls ``build_binding()``; the CPU tests call both.
"""
from __future__ import annotations

import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INCLUDE = os.path.join(ROOT, "include")
LIBDIR = os.path.join(ROOT, "slime_amd")
OUT_DIR = os.path.join(HERE, "_build")
BINDING = os.path.join(OUT_DIR, "ca_binding")
ROCM = "/opt/rocm"


def compile_header(lang: str) -> None:
    """Raises CalledProcessError with the compiler's message if the header does not
    compile alone."""
    with tempfile.TemporaryDirectory() as d:
        if lang == "c":
            src, cmd = os.path.join(d, "h.c"), ["gcc", "-std=c99"]
        else:
            src, cmd = os.path.join(d, "h.cpp"), ["g++", "-std=c++17"]
        with open(src, "w") as f:
            f.write('#include "slime_ca.h"\n')
        subprocess.run(cmd + ["-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{INCLUDE}",
                              "-fsyntax-only", src], check=True, capture_output=True, text=True)


def build_binding() -> str:
    if not os.path.exists(os.path.join(LIBDIR, "libslime_ca.so")):
        raise FileNotFoundError("slime_amd/libslime_ca.so is not built")
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = BINDING + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{INCLUDE}", f"-I{ROCM}/include", os.path.join(HERE, "ca_binding.cpp"),
           f"-L{LIBDIR}", "-lslime_ca", f"-L{ROCM}/lib", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/../../slime_amd", f"-Wl,-rpath,{ROCM}/lib", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building ca_binding failed:\n{r.stderr}")
    os.replace(tmp, BINDING)
    return BINDING


if __name__ == "__main__":
    compile_header("c")
    compile_header("c++")
    print(build_binding())
