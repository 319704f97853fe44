"""Builds libgnn_hip.so (the gfx950 HIP kernels + C ABI) in-tree.

Usage: python geometric-nn-ops_amd/build.py [--jobs N]

Each csrc/*.hip file is compiled to an object in parallel with hipcc for gfx950 only,
then linked into geometric_nn_ops_torch/_lib/libgnn_hip.so, which the package loads
with ctypes. Always recompiles (it is the "does it build" check).
"""

import argparse
import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = REPO / "include"
OUT_DIR = HERE / "geometric_nn_ops_torch" / "_lib"
LIB = OUT_DIR / "libgnn_hip.so"
BUILD_DIR = HERE / "_build"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU ops stay off: hipcc would otherwise form v_pk_{add,mul,fma}_f32
    # from ordinary float code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
# Per-source flags. The row-resident attention kernel schedules for instruction-level
# parallelism (LLVM's AMDGPU max-ilp machine scheduler): 1.5-2 us (1%) less per forward
# inside the headline step (174.1 -> 172.0 us on one box, 177.3 / 176.8 -> 175.7 / 174.6 on
# another), at the same 128 VGPRs without spills. The same strategy on trimul.hip slowed the contraction and output stages
# (+0.7 and +1.5 us) more than it sped up the projection (-0.5 us), and the
# memory-clause strategy slowed the fp32 'tf32' block (0.815 -> 0.868 ms). max-ilp on the
# backward files slowed the attention and trimul backward passes.
FILE_FLAGS = {
    "triattn_row.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = pathlib.Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def _compile(src: pathlib.Path, build_dir: pathlib.Path = BUILD_DIR, extra=()) -> pathlib.Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, ()), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False, defines=(), out: pathlib.Path | None = None) -> pathlib.Path:
    """Compile and link the library; ``defines`` (``NAME=VALUE`` strings) select the tuning
    macros of the kernels, ``out`` writes the library elsewhere (objects then go to a build
    folder of their own) -- how the measured alternatives in the kernels' comments are built."""
    lib = LIB if out is None else pathlib.Path(out).resolve()
    build_dir = BUILD_DIR if not defines and out is None else BUILD_DIR.with_name(BUILD_DIR.name + "_" + lib.stem)
    build_dir.mkdir(exist_ok=True)
    lib.parent.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 16)
    extra = [f"-D{d}" for d in defines]
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(lambda src: _compile(src, build_dir, extra), sources))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--define", action="append", default=[], metavar="NAME=VALUE",
                    help="kernel tuning macro, e.g. GNN_ROW_MAX_N=0 (tiled attention only)")
    ap.add_argument("--out", default=None, help="library path (default: the package's _lib/libgnn_hip.so)")
    args = ap.parse_args()
    build(args.jobs, verbose=True, defines=args.define, out=args.out)
    sys.exit(0)
