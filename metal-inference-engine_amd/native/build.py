"""Build librk_path.so: every HIP source in this directory, compiled ahead of time for gfx950 only.

The counterpart of the reference's scripts/build_native.sh (clang++ -framework Metal ... -shared), which builds its
one native file into build/. Here hipcc compiles each translation unit to an object and links one shared library
next to the sources, so the library travels with the tree. Usage: python native/build.py [-v]
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "librk_path.so"
PROBE_LIB = HERE / "librk_probe.so"       # measurement probes (include/rk_probe.h), not on the path
OBJ_DIR = HERE / "_obj"
SOURCES = ["rk_abi.cpp", "paged_decode.hip", "kv_cache.hip", "page_table.hip", "deltanet_step.hip", "paged_prefill.hip",
           "chunked_delta.hip", "chunked_delta_cols.hip", "deltanet_prefill.hip", "attn_prep.hip",
           "linear.hip", "decode_ops.hip"]
PROBE_SOURCES = ["probes.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# packed-fp32 VALU forms are switched off for all device code (see the header of rk_device.h)
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


# per-source additions: the bf16 delta scan splits and scales its MFMA results every chunk, so they stay in VGPRs;
# the sources that restate the reference's elementwise steps with each product and sum rounded (__fmul_rn /
# __fadd_rn, which HIP defines as the plain operators) are compiled with FMA contraction inside one expression only,
# so that hipcc's default (contraction across statements) does not fuse a rounded product into the sum after it
_ROUNDED = ["-ffp-contract=on"]
SOURCE_FLAGS = {"chunked_delta_cols.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "deltanet_step.hip": _ROUNDED,
                "decode_ops.hip": _ROUNDED, "deltanet_prefill.hip": _ROUNDED, "attn_prep.hip": _ROUNDED,
                "linear.hip": _ROUNDED}


def _compile(src: str, verbose: bool) -> Path:
    obj = OBJ_DIR / (Path(src).stem + ".o")
    cmd = [HIPCC, "-x", "hip", "-c", str(HERE / src), "-o", str(obj)] + FLAGS + SOURCE_FLAGS.get(src, [])
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 target feature and says so: not an error
    noise = [ln for ln in (r.stderr or "").splitlines() if "not a recognized feature" not in ln]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n" + "\n".join(noise))
    if verbose and noise:
        print("\n".join(noise))
    return obj


def _link(lib: Path, objs: list[Path], verbose: bool) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-o", str(tmp)] + [str(o) for o in objs] + [f"--offload-arch={ARCH}", "-fPIC"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {lib.name} failed:\n" + r.stderr)
    os.replace(tmp, lib)


def build(verbose: bool = False) -> Path:
    """Compile every source and link librk_path.so and librk_probe.so (always rebuilds). Returns the path
    library."""
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = SOURCES + PROBE_SOURCES
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = dict(zip(srcs, ex.map(lambda s: _compile(s, verbose), srcs)))
    _link(LIB, [objs[s] for s in SOURCES], verbose)
    _link(PROBE_LIB, [objs[s] for s in PROBE_SOURCES] + [objs["rk_abi.cpp"]], verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
