"""Builds libmatricxon_amd.so in-tree from csrc/*.hip with hipcc for gfx950.

    python -m matricxon_amd.build

The library is written to matricxon_amd/libmatricxon_amd.so through a temp file and a rename,
so a concurrently starting process never loads a half-written file (the pattern of the
reference's loader, app/native/library.py:70-91).
"""

import os
import re
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libmatricxon_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    # every float rounding step is explicit in the sources (bit-exact dequant and folds)
    "-ffp-contract=off",
    # no packed-FP32 instructions (v_pk_*_f32) anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # leading scalar / pointer kernel arguments arrive preloaded in SGPRs, so a kernel's first
    # memory requests need no kernel-argument load (measured: -0.25 us per 33 MB launch)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


# Sources whose kernels must use no scratch memory. mxa_bwave.hip issues loads into registers
# from inline assembly and waits for them itself; the compiler treats those registers as written
# at issue, so a spill (or any reuse of them) before the wait would read or clobber registers a
# load still writes. Such a build is refused rather than shipped.
NO_SCRATCH = {"mxa_bwave.hip"}
_RESOURCE_REMARKS = "-Rpass-analysis=kernel-resource-usage"


def scratch_users(stderr: str) -> list[str]:
    """Kernels with a nonzero 'ScratchSize' in hipcc's kernel-resource-usage remarks."""
    bad, name = [], None
    for line in stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name is not None and int(m.group(1)) > 0:
            bad.append(f"{name} ({m.group(1)} bytes/lane)")
    return bad


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build matricxon_amd)")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _jobs() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, int(os.environ.get("MAX_JOBS", "16")), 16))


def build(verbose: bool = False) -> Path:
    """Compiles every csrc/*.hip into LIB_PATH: one object per source, compiled in parallel into
    _build/, then one link. Raises RuntimeError with the compiler output on failure."""
    from concurrent.futures import ThreadPoolExecutor

    obj_dir = PKG_DIR.parent / "_build" / "csrc"
    obj_dir.mkdir(parents=True, exist_ok=True)
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]

    def compile_one(src: Path) -> tuple[Path, subprocess.CompletedProcess]:
        obj = obj_dir / (src.stem + ".o")
        extra = [_RESOURCE_REMARKS] if src.name in NO_SCRATCH else []
        cmd = [hipcc(), *compile_flags, *extra, "-c", "-o", str(obj), str(src)]
        if verbose:
            print(" ".join(cmd), flush=True)
        return obj, subprocess.run(cmd, capture_output=True, text=True)

    srcs = sources()
    with ThreadPoolExecutor(_jobs()) as pool:
        results = list(pool.map(compile_one, srcs))
    errors = [r.stderr for _, r in results if r.returncode != 0]
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n".join(e[-8000:] for e in errors))
    for src, (_, r) in zip(srcs, results):
        if src.name in NO_SCRATCH:
            bad = scratch_users(r.stderr)
            if bad:
                raise RuntimeError(f"{src.name}: kernels that must not use scratch do: " + ", ".join(bad))
    fd, tmp = tempfile.mkstemp(dir=PKG_DIR, suffix=".so.tmp")
    os.close(fd)
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp,
           *(str(o) for o, _ in results)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        Path(tmp).unlink(missing_ok=True)
        raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.chmod(tmp, 0o755)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
