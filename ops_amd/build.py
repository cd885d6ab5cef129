"""Build libsfa.so (HIP, gfx950) in-tree with hipcc.

``python -m ops_amd.build`` compiles every ``csrc/*.hip`` into
``ops_amd/libsfa.so``.  Flags: -O3, gfx950 only, and packed-fp32 ops disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``) so hipcc never emits
v_pk_{add,mul,fma}_f32.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libsfa.so"
ARCH = os.environ.get("SFA_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wno-unused-result",
    # MFMA builtins in VGPR form: the large O^T accumulators are pinned to
    # AGPRs explicitly, everything else stays in VGPRs
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.sep not in c or os.path.exists(c)):
            return c
    return "hipcc"


def sources():
    return sorted(str(p) for p in CSRC.glob("*.hip"))


def build(verbose: bool = False, extra=None) -> Path:
    """Compile the library; raises CalledProcessError on a compile failure."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *(extra or []), "-I", str(HERE.parent / "include"), *sources(), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise subprocess.CalledProcessError(res.returncode, cmd, res.stdout, res.stderr)
    os.replace(tmp, LIB)
    return LIB


PROBE_SRC = CSRC / "probe" / "sfa_probe.hip"
PROBE_LIB = HERE / "libsfa_probe.so"


def build_probe(verbose: bool = False) -> Path:
    """Compile the measurement-only probe library (libsfa_probe.so: the
    decode's gathers without their MFMA work, for ``bench.py --probe``)."""
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(HERE.parent / "include"), str(PROBE_SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise subprocess.CalledProcessError(res.returncode, cmd, res.stdout, res.stderr)
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def resource_usage() -> str:
    """Markdown table of every kernel's registers, scratch (spills), LDS and
    occupancy as the compiler reports them (-Rpass-analysis=kernel-resource-usage,
    one device-only compile per source)."""
    import re
    rows = []
    for src in sources():
        cmd = [hipcc(), *[f for f in HIPCC_FLAGS if f not in ("-shared", "-fPIC")], "--cuda-device-only", "-c",
               "-Rpass-analysis=kernel-resource-usage", "-I", str(HERE.parent / "include"), src, "-o", os.devnull]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stderr)
            raise subprocess.CalledProcessError(res.returncode, cmd)
        cur = None
        for line in res.stderr.splitlines():
            m = re.search(r"remark: (?:\S+: )?\s*([A-Za-z ]+?)(?: \[[^]]*\])?: (\S+)(?: \[-Rpass)", line)
            if not m:
                continue
            key, val = m.group(1).strip(), m.group(2)
            if key == "Function Name":
                cur = {"kernel": val, "file": os.path.basename(src)}
                rows.append(cur)
            elif cur is not None:
                cur[key] = val
    out = ["| kernel (mangled) | file | VGPRs | AGPRs | SGPRs | scratch B/lane | LDS B | waves/SIMD |",
           "|---|---|---|---|---|---|---|---|"]
    for r in rows:
        out.append(f"| `{r['kernel']}` | {r['file']} | {r.get('VGPRs', '?')} | {r.get('AGPRs', '?')} | "
                   f"{r.get('TotalSGPRs', '?')} | {r.get('ScratchSize', '?')} | {r.get('LDS Size', '?')} | "
                   f"{r.get('Occupancy', '?')} |")
    return "\n".join(out)


if __name__ == "__main__":
    if "--resource-usage" in sys.argv:
        print(resource_usage())
    else:
        print(build(verbose=True))
        print(build_probe(verbose=True))
