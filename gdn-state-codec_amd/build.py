"""Build the gfx950 codec library in-tree.

Compiles every HIP/C++ source under ``csrc/`` with hipcc for gfx950 into
``lib/libstatecentric_gdn_state_codec.so`` and adds the library file names
the reference's ctypes loader resolves (``src/gdn_state_codec/runtime.py:55-237``)
as symlinks to it, so ``GDN_STATE_CODEC_LIBRARY_DIR=<package>/lib`` is a
drop-in library directory.

Usage: ``python gdn-state-codec_amd/build.py`` (also run by
``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "lib"
OBJ_DIR = LIB_DIR / "obj"
LIBRARY_NAME = "libstatecentric_gdn_state_codec.so"
# Probes (csrc/bench/): HBM bandwidth for bench.py and the wavefront-exchange
# self-check for the tests; not part of the C-ABI.
PROBE_LIBRARY_NAME = "libgdn_state_codec_hbm_probe.so"

# Reference library names (runtime.py:55-62, 72, 101, 131, 154, 182, 202, 224)
# whose hot-path symbols this library exports.
REFERENCE_LIBRARY_NAMES = (
    "libstatecentric_gdn_state_codec_smoothing_kernel.so",
    "libstatecentric_gdn_state_codec_quantize_kernel.so",
    "libstatecentric_gdn_state_codec_dequantize_kernel.so",
    "libstatecentric_gdn_state_codec_provider_runtime.so",
    "libstatecentric_gdn_state_codec_encoded_projection_kernel.so",
    "libstatecentric_gdn_state_codec_windowed_gdn_step_kernel.so",
    "libstatecentric_gdn_state_codec_window_boundary_kernel.so",
    "libstatecentric_gdn_state_codec_bf16_cube_matmul_kernel.so",
    "libstatecentric_gdn_state_codec_int8_cube_matmul_kernel.so",
    "libstatecentric_gdn_state_codec_boundary_runtime.so",
    "libstatecentric_gdn_state_codec_decode_runtime.so",
)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Exact IEEE semantics for the bit-exact codec: no implicit contraction.
    "-ffp-contract=off",
    # No packed fp32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    f"-I{REPO_ROOT / 'include'}",
    f"-I{CSRC}",
]


def _sources() -> list[Path]:
    return sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp"))


def _compile(source: Path) -> Path:
    obj = OBJ_DIR / (source.parent.name + "_" + source.stem + source.suffix.replace(".", "_") + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)
    return obj


def _link(objects: list[Path], name: str) -> Path:
    target = LIB_DIR / name
    tmp = LIB_DIR / (name + ".tmp")
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC",
            *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, target)
    return target


def build(verbose: bool = True) -> Path:
    """Compile all sources and link the shared libraries; returns the codec's."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    sources = _sources()
    probes = sorted((CSRC / "bench").glob("*.hip"))
    jobs = min(len(sources) + len(probes), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(jobs, 1)) as pool:
        objects = list(pool.map(_compile, sources))
        probe_objects = list(pool.map(_compile, probes))
    target = _link(objects, LIBRARY_NAME)
    if probe_objects:
        _link(probe_objects, PROBE_LIBRARY_NAME)
    for name in REFERENCE_LIBRARY_NAMES:
        alias = LIB_DIR / name
        if alias.is_symlink() or alias.exists():
            alias.unlink()
        alias.symlink_to(LIBRARY_NAME)
    shutil.rmtree(OBJ_DIR, ignore_errors=True)
    if verbose:
        print(f"built {target}")
    return target


if __name__ == "__main__":
    build()
