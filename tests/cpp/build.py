"""Build the C/C++ callers the GPU tests run (test infrastructure):

    python tests/cpp/build.py

w8a8_c_harness      plain C99 over include/w8a8.h and the HIP runtime's C API
kitchen_bridge_test C++ over LibTorch, driving libimagine_kitchen.so through
                    dlopen the way the reference crate drives its bridge
Both binaries land next to their sources (git-ignored) and travel with the
tree; __graft_entry__.build() runs this after building the libraries.
"""
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from imagine_amd import build as B  # noqa: E402


def run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed:\n{r.stderr[-4000:]}")


def build():
    rocm = Path(B.hipcc()).resolve().parents[1]
    pkg = ROOT / "imagine_amd"
    run(["gcc", "-O2", "-std=c99", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{rocm / 'include'}", f"-I{ROOT / 'include'}",
         str(HERE / "w8a8_c_harness.c"), "-o", str(HERE / "w8a8_c_harness"), f"-L{pkg}", "-lw8a8_hip",
         f"-L{rocm / 'lib'}", "-lamdhip64", "-ldl", f"-Wl,-rpath,{pkg}", f"-Wl,-rpath,{rocm / 'lib'}"])
    t = B.torch_dir()
    run(["g++", "-O1", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{t / 'include'}",
         f"-I{t / 'include' / 'torch' / 'csrc' / 'api' / 'include'}", f"-I{rocm / 'include'}",
         str(HERE / "kitchen_bridge_test.cpp"), "-o", str(HERE / "kitchen_bridge_test"), f"-L{t / 'lib'}",
         "-Wl,--no-as-needed", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10", "-lc10_hip", "-Wl,--as-needed",
         f"-L{rocm / 'lib'}", "-lamdhip64", "-ldl", f"-Wl,-rpath,{t / 'lib'}", f"-Wl,-rpath,{rocm / 'lib'}"])
    return [HERE / "w8a8_c_harness", HERE / "kitchen_bridge_test"]


if __name__ == "__main__":
    for p in build():
        print(p)
