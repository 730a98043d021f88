"""Compile libkvip_hip.so for gfx950 with hipcc.

Mirrors the role of the reference's content-keyed library build
(python/kvip/runtime/build.py:40-91) without CMake: every ``kvip_amd/csrc/*.hip``
file is compiled and linked into one in-tree shared library, which travels with
the source tree (no JIT cache, no site-packages install).
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parents[1]
ROOT = PACKAGE.parent
SOURCES = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
OUTPUT = PACKAGE / "_lib" / "libkvip_hip.so"
OBJECTS = PACKAGE / "_lib" / "_build"
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for every HIP file (hipcc's host pass warns
# that it does not know the feature; that warning is harmless).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-mcode-object-version=5",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # MFMA accumulators in VGPRs (gfx950 has a unified register file): the epilogue then
    # reads them without v_accvgpr_read moves.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: libkvip_hip.so needs ROCm's hipcc to build")
    return path


def source_files():
    return sorted(SOURCES.glob("*.hip"))


def source_digest() -> str:
    digest = hashlib.sha256()
    for path in sorted(list(SOURCES.glob("*")) + list(INCLUDE.glob("*.h"))):
        if path.is_file():
            digest.update(path.name.encode())
            digest.update(path.read_bytes())
    digest.update(" ".join(HIPCC_FLAGS).encode())
    return digest.hexdigest()


def files_digest(paths) -> str:
    """Digest of the named files (paths relative to the repository root) and the compile
    flags: identifies the sources a measurement of particular kernels was taken on."""
    digest = hashlib.sha256()
    for rel in sorted(paths):
        path = ROOT / rel
        digest.update(rel.encode())
        digest.update(path.read_bytes() if path.is_file() else b"<missing>")
    digest.update(" ".join(HIPCC_FLAGS).encode())
    return digest.hexdigest()


def _compile(source: Path, jobs_dir: Path) -> Path:
    obj = jobs_dir / (source.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{SOURCES}", "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name} ({result.returncode}):\n{result.stderr[-6000:]}")
    return obj


def build_libraries(force: bool = True, verbose: bool = False) -> Path:
    """Compile every HIP source into kvip_amd/_lib/libkvip_hip.so: one object per source,
    compiled in parallel (each translation unit carries its own gfx950 code object), then
    one shared-library link.

    force=False skips the compile when the stamped source digest matches."""
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    stamp = OUTPUT.with_suffix(".sha256")
    digest = source_digest()
    if not force and OUTPUT.exists() and stamp.exists() and stamp.read_text() == digest:
        return OUTPUT
    jobs_dir = OBJECTS / f"p{os.getpid()}"
    jobs_dir.mkdir(parents=True, exist_ok=True)
    try:
        sources = source_files()
        workers = max(1, min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
        with ThreadPoolExecutor(workers) as pool:
            objects = list(pool.map(lambda src: _compile(src, jobs_dir), sources))
        tmp = OUTPUT.with_name(OUTPUT.name + f".tmp{os.getpid()}")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"hipcc link failed ({result.returncode}):\n{result.stderr[-6000:]}")
        if verbose and result.stderr:
            print(result.stderr)
        os.replace(tmp, OUTPUT)
    finally:
        shutil.rmtree(jobs_dir, ignore_errors=True)
    stamp.write_text(digest)
    return OUTPUT
