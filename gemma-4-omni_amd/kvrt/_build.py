"""Build libkvrt.so (gfx950) in-tree with hipcc.

The library is compiled from ``csrc/kvrt_kernels.hip`` (kernels) and
``csrc/kvrt_runtime.hip`` (host runtime, C ABI in ``include/kvrt.h``). The
build also compiles ``csrc/kvrt_coherence_probe.hip`` to assembly (never
linked) and fails if the coherent-access helpers lower differently from what
the single-launch decode merge relies on.
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


# The single-launch decode merge exchanges partials and arrival counts between
# workgroups on different XCDs through relaxed agent-scope atomics only
# (kvrt_device.h), and is correct because gfx950 lowers them to device-scope
# accesses: stores written through the XCD's L2 and loads read past it (sc1),
# the counter an L2 atomic add returning its old value (sc0), with no L2
# write-back or invalidate. kvrt_coherence_probe.hip compiles each helper
# alone; this is the memory-instruction sequence (opcode, cache-policy bits)
# each probe kernel must lower to, the helper's own access first and, for the
# loads and the counter, the plain store of the value read.
COHERENCE_PROBE = CSRC / "kvrt_coherence_probe.hip"
COHERENCE_LOWERING = {
    "kvrt_probe_store_f32": [("global_store_dword", {"sc1"})],
    "kvrt_probe_store_f32x2": [("global_store_dwordx2", {"sc1"})],
    "kvrt_probe_store16": [("global_store_dwordx2", {"sc1"}), ("global_store_dwordx2", {"sc1"})],
    "kvrt_probe_load_f32": [("global_load_dword", {"sc1"}), ("global_store_dword", set())],
    "kvrt_probe_load_f32x2": [("global_load_dwordx2", {"sc1"}), ("global_store_dwordx2", set())],
    "kvrt_probe_arrive": [("global_atomic_add", {"sc0"}), ("global_store_dword", set())],
    "kvrt_probe_clear": [("global_store_dword", {"sc1"})],
}
_MEM_PREFIXES = ("global_", "buffer_", "flat_", "scratch_")
_POLICY_BITS = {"sc0", "sc1", "nt"}


def memory_ops(asm: str) -> dict[str, list[tuple[str, set[str]]]]:
    """Memory instructions of each kernel in a device assembly listing, as
    (opcode, cache-policy bits) in program order."""
    ops: dict[str, list[tuple[str, set[str]]]] = {}
    cur = None
    for line in asm.splitlines():
        label = re.match(r"^([A-Za-z_][\w.]*):", line)
        if label:
            cur = label.group(1)
            ops[cur] = []
            continue
        toks = line.split(";")[0].split()
        if cur is None or not toks or not toks[0].startswith(_MEM_PREFIXES):
            continue
        ops[cur].append((toks[0], {t.rstrip(",") for t in toks[1:]} & _POLICY_BITS))
    return ops


def coherence_errors(asm: str) -> list[str]:
    """Differences between the probe kernels' lowering and COHERENCE_LOWERING."""
    ops = memory_ops(asm)
    errs = []
    for name, want in COHERENCE_LOWERING.items():
        got = ops.get(name)
        if got is None:
            errs.append(f"{name}: not found in the probe's assembly")
        elif got != want:
            errs.append(f"{name}: lowered to {got}, expected {want}")
    for name, got in ops.items():
        extra = [op for op, _ in got if op.startswith(("buffer_wbl2", "buffer_inv", "buffer_wbinvl1"))]
        if name in COHERENCE_LOWERING and extra:
            errs.append(f"{name}: cache maintenance {extra} around a relaxed access")
    return errs


def coherence_probe_asm() -> str:
    """kvrt_coherence_probe.hip compiled to gfx950 assembly with the library's flags."""
    with tempfile.TemporaryDirectory(prefix="kvrt_probe_") as tmp:
        out = Path(tmp) / "probe.s"
        cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", "--offload-device-only", "-S", str(COHERENCE_PROBE),
               "-o", str(out)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {COHERENCE_PROBE.name}:\n{res.stderr}")
        return out.read_text()


def check_coherence_lowering() -> None:
    """Refuse a compiler that lowers the coherent-access helpers other than
    the single-launch merge relies on."""
    errs = coherence_errors(coherence_probe_asm())
    if errs:
        raise RuntimeError("agent-scope coherent accesses lower differently from what the single-launch "
                           "decode merge relies on:\n  " + "\n  ".join(errs))


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link libkvrt.so next to this file."""
    with tempfile.TemporaryDirectory(prefix="kvrt_build_") as tmp:
        objs = [Path(tmp) / (Path(s).stem + ".o") for s in SOURCES]
        with ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as pool:
            futs = [pool.submit(_compile, CSRC / s, o) for s, o in zip(SOURCES, objs)]
            probe = pool.submit(check_coherence_lowering)
            resources: dict[str, dict[str, str]] = {}
            for f in futs:
                resources.update(f.result())
            probe.result()
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
