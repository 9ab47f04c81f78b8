"""Builds the HIP shared library in-tree: ``liteinfer_amd/_lib/libliteinfer_amd.so``.

Every ``csrc/*.hip`` file is compiled for gfx950 by ``hipcc`` and linked into
one shared library with a plain C ABI (``include/liteinfer_amd.h``). The
library is loaded with ctypes, so nothing here depends on torch's extension
machinery; it links the HIP runtime by soname, which resolves to the copy the
process already has loaded when torch was imported first.

Run as ``python -m liteinfer_amd._build``.
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_PATH = LIB_DIR / "libliteinfer_amd.so"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"

OFFLOAD_ARCH = "gfx950"

# Packed fp32 instructions stay off: some of their forms have given wrong
# results on these machines with no error raised.
DEVICE_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-honor-nans",
    "-Wall",
    "-Wno-unused-function",
]


# Per-source extra flags. prefill_mfma.hip: its persistent kernel claims the
# next unit with an atomic whose old value it reads only at the unit's end;
# the wave-level atomic optimizer would read it back at once, stalling the
# wave on every load in flight.
SOURCE_FLAGS = {
    "prefill_mfma.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def source_hash() -> str:
    """16 hex digits of SHA-256 over every source and header and the compile flags.

    The build passes it into the library (``li_build_id``); the loader
    recomputes it from the files beside the package and refuses a mismatch.
    """
    h = hashlib.sha256()
    files = sorted(p for p in CSRC_DIR.iterdir() if p.is_file() and p.suffix in (".hip", ".h", ".cpp"))
    files += sorted(INCLUDE_DIR.glob("*.h"))
    for path in files:
        h.update(path.name.encode() + b"\0" + path.read_bytes() + b"\0")
    h.update(repr((DEVICE_FLAGS, sorted(SOURCE_FLAGS.items()))).encode())
    return h.hexdigest()[:16]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found: set ROCM_PATH or put hipcc on PATH")
    return found


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def _compile(src: Path, obj: Path, build_id: str) -> None:
    cmd = [hipcc(), *DEVICE_FLAGS, *SOURCE_FLAGS.get(src.name, []), f'-DLI_BUILD_ID="{build_id}"',
           "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that
    # warning is harmless and is the only output dropped.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every source and link the library. Always rebuilds."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    build_id = source_hash()
    with tempfile.TemporaryDirectory(prefix="liteinfer_amd_build_") as tmp:
        objs = []
        jobs = []
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
            for src in sources():
                obj = Path(tmp) / (src.stem + ".o")
                objs.append(obj)
                jobs.append(pool.submit(_compile, src, obj, build_id))
            for job in jobs:
                job.result()
        out_tmp = LIB_DIR / (LIB_PATH.name + ".tmp")
        cmd = [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(out_tmp), *map(str, objs)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stderr}")
        os.replace(out_tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
