#!/usr/bin/env python3
"""Writes the golden fixtures of the sparse-attention oracle.

``sfa_golden.npz`` holds, per case, small seeded inputs and the outputs the
CPU oracle (``oracle/sfa_oracle.py``) computes from them in float64: ``out``,
``lse``, ``dq``, ``dk``, ``dv`` (and ``dsink`` when the case has a sink).
``MANIFEST.json`` records each case's seed and shapes and the file's sha256.

The reference ships no vectors of its own (its tree holds only SFA.py and
README.md), so these fixtures are the drift guard of the oracle's
restatement of SFA.py:359-480 (forward), 590-610 (δ), 613-853 (dQ, dK/dV)
and 964-970 (dsink): ``tests/test_golden.py`` re-derives every stored output
from the stored inputs and fails if the oracle's results move, and
``tests/test_gpu_golden.py`` holds the HIP path to the same vectors.

Inputs come from numpy's PCG64 generator (float32 N(0,1) values; the bf16
cases round them to bf16 first, so the stored float32 values are exact in
bf16).  Index rows mix causal sampling with interior -1 padding and
out-of-range ids.  Run ``python tests/golden/make_golden.py`` to rewrite
both files (only when a deliberate change of the oracle calls for it).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

NPZ = os.path.join(HERE, "sfa_golden.npz")
MANIFEST = os.path.join(HERE, "MANIFEST.json")

# name -> parameters.  'idx' recipes: 'causal' = query t samples min(K, t+1)
# distinct keys of [0, t] (random order), then -1 padding; 'mixed' = ids
# drawn from [-3, Skv + 3) (so -1, < -1 and >= Skv all occur), one row fully
# invalid.
CASES = {
    "tiny_causal_fp32": dict(seed=11, B=1, S=32, Skv=32, Hq=4, Hkv=1, Dqk=16, Dv=16, K=8, idx="causal",
                             bf16=False, kv_lens=None, sink=False),
    "gqa_kvlens_sink_fp32": dict(seed=12, B=2, S=24, Skv=40, Hq=6, Hkv=2, Dqk=32, Dv=24, K=12, idx="mixed",
                                 bf16=False, kv_lens=[40, 29], sink=True),
    "d128_g2_bf16": dict(seed=13, B=1, S=32, Skv=32, Hq=2, Hkv=1, Dqk=128, Dv=128, K=16, idx="causal",
                         bf16=True, kv_lens=None, sink=False),
}


def _bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), as float32."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def make_inputs(c: dict) -> dict:
    rng = np.random.Generator(np.random.PCG64(c["seed"]))
    B, S, Skv, Hq, Hkv, Dqk, Dv, K = (c[n] for n in ("B", "S", "Skv", "Hq", "Hkv", "Dqk", "Dv", "K"))
    x = {
        "q": rng.standard_normal((B, S, Hq, Dqk), dtype=np.float32),
        "k": rng.standard_normal((B, Skv, Hkv, Dqk), dtype=np.float32),
        "v": rng.standard_normal((B, Skv, Hkv, Dv), dtype=np.float32),
        "dout": rng.standard_normal((B, S, Hq, Dv), dtype=np.float32),
    }
    if c["bf16"]:
        x = {n: _bf16_round(a) for n, a in x.items()}
    idx = np.full((B, S, Hkv, K), -1, dtype=np.int32)
    if c["idx"] == "causal":
        for b in range(B):
            for t in range(S):
                for g in range(Hkv):
                    n = min(K, t + 1)
                    idx[b, t, g, :n] = rng.permutation(t + 1)[:n]
    else:
        idx[:] = rng.integers(-3, Skv + 3, size=idx.shape, dtype=np.int32)
        idx[-1, S // 2] = -1
    x["idx"] = idx
    if c["kv_lens"] is not None:
        x["kv_lens"] = np.asarray(c["kv_lens"], dtype=np.int32)
    if c["sink"]:
        x["sink"] = rng.standard_normal((Hq,), dtype=np.float32)
    x["scale"] = np.asarray(1.0 / np.sqrt(Dqk), dtype=np.float64)
    return x


def oracle_outputs(x: dict) -> dict:
    """float64 oracle forward + backward on the case's inputs."""
    import torch
    from oracle.sfa_oracle import sfa_backward, sfa_forward

    t = {n: torch.from_numpy(np.ascontiguousarray(a)) for n, a in x.items()}
    scale = float(x["scale"])
    kv_lens = t.get("kv_lens")
    sink = t.get("sink")
    out, lse = sfa_forward(t["q"], t["k"], t["v"], t["idx"], scale, kv_lens=kv_lens, sink=sink, dtype=torch.float64)
    dq, dk, dv, dsink = sfa_backward(t["q"], t["k"], t["v"], t["idx"], out, lse, t["dout"], scale, kv_lens=kv_lens,
                                     sink=sink, dtype=torch.float64)
    y = {"out": out, "lse": lse, "dq": dq, "dk": dk, "dv": dv}
    if dsink is not None:
        y["dsink"] = dsink
    return {n: a.numpy() for n, a in y.items()}


def sha256(path: str) -> str:
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def main() -> None:
    arrays, manifest = {}, {"file": os.path.basename(NPZ), "generator": "numpy PCG64, float32 standard_normal",
                            "oracle": "oracle/sfa_oracle.py sfa_forward + sfa_backward, float64", "cases": {}}
    for name, c in CASES.items():
        x = make_inputs(c)
        y = oracle_outputs(x)
        for n, a in {**x, **y}.items():
            arrays[f"{name}/{n}"] = a
        manifest["cases"][name] = {**c, "inputs": sorted(x), "outputs": sorted(y),
                                   "valid_pairs": int(((x["idx"] >= 0) & (x["idx"] < (
                                       np.asarray(c["kv_lens"]).reshape(-1, 1, 1, 1) if c["kv_lens"] is not None
                                       else c["Skv"]))).sum())}
    np.savez_compressed(NPZ, **arrays)
    manifest["sha256"] = sha256(NPZ)
    with open(MANIFEST, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {NPZ} ({os.path.getsize(NPZ)} bytes), sha256 {manifest['sha256']}")


if __name__ == "__main__":
    main()
