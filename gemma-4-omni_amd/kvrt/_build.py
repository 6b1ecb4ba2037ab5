"""Build libkvrt.so (gfx950) in-tree with hipcc.

The library is compiled from ``csrc/kvrt_kernels.hip`` (kernels) and
``csrc/kvrt_runtime.hip`` (host runtime, C ABI in ``include/kvrt.h``).
"""
from __future__ import annotations

import json
import os
import re
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parent.parent / "include"
LIB_PATH = PKG_DIR / "libkvrt.so"
SOURCES = ("kvrt_kernels.hip", "kvrt_runtime.hip")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed FP32 VALU forms are kept out of every code object.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # MFMA accumulators live in ordinary VGPRs. With the default AGPR form the
    # prefill tile loop copied its output accumulators between the two
    # register files every tile (72 v_accvgpr moves per 32-key tile at D 128);
    # the VGPR form drops them and raises occupancy of several decode and
    # prefill instantiations (talker prefill 26.4 -> 23.8 us per launch).
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall",
    "-Wno-unused-function",
    # flowing off the end of a value-returning function is undefined (a
    # launcher lambda that did so crashed the host): refuse to build it
    "-Werror=return-type",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the kvrt HIP library cannot be built")


RESOURCES_PATH = PKG_DIR / "kernel_resources.json"
_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]"
                     r"|LDS Size \[bytes/block\]):\s+(\S+)")


def _resources(stderr: str) -> dict[str, dict[str, str]]:
    """Per-kernel VGPR / scratch / LDS / occupancy from the compiler's resource remarks."""
    out: dict[str, dict[str, str]] = {}
    name = None
    for m in _REMARK.finditer(stderr):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            name = val
            out[name] = {}
        elif name is not None:
            out[name][key.split(" ")[0]] = val
    return out


def _compile(src: Path, obj: Path) -> dict[str, dict[str, str]]:
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj),
           "-Rpass-analysis=kernel-resource-usage"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in res.stderr.splitlines() if noise not in l and "remark" not in l)
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return _resources(res.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link libkvrt.so next to this file."""
    with tempfile.TemporaryDirectory(prefix="kvrt_build_") as tmp:
        objs = [Path(tmp) / (Path(s).stem + ".o") for s in SOURCES]
        with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
            futs = [pool.submit(_compile, CSRC / s, o) for s, o in zip(SOURCES, objs)]
            resources: dict[str, dict[str, str]] = {}
            for f in futs:
                resources.update(f.result())
        # Every kernel of the hot path must run from registers and LDS: scratch
        # (private segment) use means spilled registers or a by-value kernel
        # argument copied to memory, both of which cost a memory round trip per use.
        spilled = {k: v["ScratchSize"] for k, v in resources.items() if v.get("ScratchSize", "0") != "0"}
        if spilled:
            raise RuntimeError(f"kernels using scratch memory: {spilled}")
        RESOURCES_PATH.write_text(json.dumps(resources, indent=1, sort_keys=True) + "\n")
        tmp_lib = Path(tmp) / "libkvrt.so"
        cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp_lib)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link of libkvrt.so failed:\n{res.stderr}")
        shutil.move(str(tmp_lib), str(LIB_PATH))
    if verbose:
        print(f"[kvrt] built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
