"""Builds libdrama3_moe.so (gfx950) from the HIP sources beside this file, in-tree at drama3/_lib/.

    python comfyui-drama3_amd/csrc/build.py

The library links against the HIP runtime by its soname (libamdhip64.so.7); the Python loader imports torch first,
so the library binds to the runtime torch already loaded and shares its streams.
"""
import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
PACKAGE = HERE.parent / "drama3"
OUT_DIR = PACKAGE / "_lib"
LIB = OUT_DIR / "libdrama3_moe.so"
ROCM = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-mcode-object-version=5",
    # packed fp32 instructions stay off: hipcc would otherwise form them from float code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def sources():
    return sorted(HERE.glob("*.hip"))


def _compile(src, obj):
    cmd = [str(HIPCC), *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in (proc.stderr or "").splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    return err


def build(verbose=False):
    """Compile every source and link the library; returns its path. Always rebuilds."""
    if not HIPCC.exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    work = HERE / "_build"
    work.mkdir(exist_ok=True)
    objs = [work / (src.stem + ".o") for src in sources()]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(objs))) as pool:
        for src, warnings in zip(sources(), pool.map(_compile, sources(), objs)):
            if verbose and warnings.strip():
                print(f"[{src.name}]\n{warnings}", file=sys.stderr)
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [str(HIPCC), "-shared", "-fPIC", "--offload-arch=gfx950", *[str(o) for o in objs], "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    shutil.rmtree(work, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
