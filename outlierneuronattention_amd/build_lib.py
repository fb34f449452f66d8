"""Build ``libhofa.so`` (all HIP sources under ``csrc/``) for gfx950 with hipcc.

``python -m outlierneuronattention_amd.build_lib`` or ``build()``.  Objects go
to ``_build/`` next to this file; the library is written in-tree so it travels
with the source tree and is found without any install step.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libhofa.so")
ARCH = "gfx950"

CXXFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Packed fp32 VALU ops stay off: hand-written or compiler-formed packed
    # fp32 arithmetic is not used anywhere in this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    return os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


# Sources compiled once per entry, each with its own defines; the key is the
# file name.  The GLA backward's launch templates are instantiated one
# (dtype, head dim, decay form) triple per object so the heavy kernels build
# in parallel (the pairs must match HOFA_GLA_BWD_FOR_EACH in
# hofa_gla_bwd_kernels.h).
VARIANTS = {
    "hofa_gla_bwd_inst.hip": [
        (f"{dt.lower()}_d{d}_g{g}", [f"-DHOFA_INST_DT=HOFA_{dt}", f"-DHOFA_INST_D={d}", f"-DHOFA_INST_GEN={g}"])
        for d in (128, 64) for dt in ("BF16", "F32", "F16") for g in (0, 1)
    ],
}


def _jobs() -> list[tuple[str, str, list[str]]]:
    """(source, object, extra flags) for every object of the library."""
    out = []
    for src in sorted(glob.glob(os.path.join(CSRC, "*.hip"))):
        name = os.path.basename(src)
        stem = name[: -len(".hip")]
        for tag, flags in VARIANTS.get(name, [("", [])]):
            obj = os.path.join(BUILD, f"{stem}_{tag}.o" if tag else f"{stem}.o")
            out.append((src, obj, flags))
    # longest compiles first
    out.sort(key=lambda j: (0 if j[2] else 1, j[1]))
    return out


def _stale(src: str, obj: str) -> bool:
    """True when obj is missing or older than its source, any csrc header or
    the C-ABI header (include/*.h, which defines the argument structs)."""
    if not os.path.exists(obj):
        return True
    deps = [src, *glob.glob(os.path.join(CSRC, "*.h")), *glob.glob(os.path.join(INCLUDE, "*.h")),
            os.path.abspath(__file__)]
    return os.path.getmtime(obj) < max(os.path.getmtime(d) for d in deps)


def _compile(job: tuple[str, str, list[str]], incremental: bool = False) -> str:
    src, obj, flags = job
    if incremental and not _stale(src, obj):
        return obj
    cmd = [hipcc(), *CXXFLAGS, *flags, "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{p.stdout}\n{p.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False, incremental: bool = False) -> str:
    """Compile every object and link libhofa.so.  incremental=True skips
    objects newer than their sources (a developer convenience; the default
    recompiles everything)."""
    os.makedirs(BUILD, exist_ok=True)
    work = _jobs()
    jobs = jobs or min(len(work), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda j: _compile(j, incremental), work))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stdout}\n{p.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(objs)} objects")
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv[1:])
    sys.exit(0)
