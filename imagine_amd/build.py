"""Build libw8a8_hip.so in-tree with hipcc for gfx950.

    python -m imagine_amd.build            # or: python imagine_amd/build.py

Each .hip source compiles to its own object in parallel, then one link.
The GELU lookup tables (imagine_amd/gelu_tables.py) are generated into the
build directory first.
Flags: -O3, IEEE float (no fast-math; contractions only where fmaf is
written), packed-fp32 instructions disabled.
"""
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libw8a8_hip.so"
SOURCES = ["w8a8_gemm_f32.hip", "w8a8_gemm_bf16.hip", "w8a8_gemm_f16.hip", "w8a8_gemm.hip", "w8a8_quant.hip",
           "w8a8_glue.hip", "w8a8_convrot.hip", "w8a8_gemv.hip", "w8a8_api.hip", "w8a8_noalloc.hip"]
ARCH = os.environ.get("W8A8_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
        "-fno-fast-math", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{ROOT / 'include'}", "-Wall", "-Wno-unused-function",
    ]


BRIDGE = PKG / "libimagine_kitchen.so"


def torch_dir():
    """LibTorch of this image (headers and libraries), located without importing torch."""
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        raise RuntimeError("the kitchen bridge needs LibTorch headers (the torch package)")
    return Path(list(spec.submodule_search_locations)[0])


def build_bridge(verbose=False):
    """libimagine_kitchen.so: the reference bridge's imagine_kitchen_call for the
    W8A8 names, over libw8a8_hip.so (g++, LibTorch headers for at::Tensor)."""
    t = torch_dir()
    rocm = Path(hipcc()).resolve().parents[1]
    with tempfile.TemporaryDirectory(prefix="w8a8_bridge_") as tmp:
        out = Path(tmp) / BRIDGE.name
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__",
               f"-I{t / 'include'}", f"-I{t / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
               f"-I{rocm / 'include'}", f"-I{ROOT / 'include'}", str(CSRC / "kitchen_bridge.cpp"), "-o", str(out),
               f"-L{PKG}", "-lw8a8_hip", f"-L{t / 'lib'}", "-lc10", "-ltorch_cpu", f"-L{rocm / 'lib'}",
               "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{t / 'lib'}", f"-Wl,-rpath,{rocm / 'lib'}"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"kitchen bridge build failed:\n{r.stderr[-4000:]}")
        if verbose and r.stderr.strip():
            print(r.stderr, file=sys.stderr)
        shutil.copy2(out, BRIDGE.with_suffix(".so.tmp"))
        os.replace(BRIDGE.with_suffix(".so.tmp"), BRIDGE)
    return BRIDGE


def build(verbose=False, extra=()):
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="w8a8_build_") as tmp:
        # generated sources: the GELU lookup tables
        sys.path.insert(0, str(ROOT))
        from imagine_amd import gelu_tables
        (Path(tmp) / "w8a8_gelu_tables.h").write_text(gelu_tables.header_text())

        def compile_one(src):
            obj = Path(tmp) / (Path(src).stem + ".o")
            cmd = [cc, *flags(), f"-I{tmp}", *extra, "-c", str(CSRC / src), "-o", str(obj)]
            r = subprocess.run(cmd, capture_output=True, text=True)
            noise = "is not a recognized feature for this target"
            err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src}:\n{err}")
            if verbose and err.strip():
                print(err, file=sys.stderr)
            return obj

        with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
            objs = list(ex.map(compile_one, SOURCES))
        tmp_lib = Path(tmp) / LIB.name
        # -z defs: a kernel whose host launch stub the compiler dropped fails here,
        # not at load time
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *map(str, objs), "-o", str(tmp_lib)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr}")
        shutil.copy2(tmp_lib, LIB.with_suffix(".so.tmp"))
        os.replace(LIB.with_suffix(".so.tmp"), LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_bridge(verbose="-v" in sys.argv))
