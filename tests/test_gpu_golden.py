"""The HIP path (through libsfa's C ABI) against the committed golden
fixtures (float64 oracle outputs on seeded inputs, tests/golden/).  Bars:
O max-abs <= 2e-2, LSE abs <= 1e-3, dQ/dK/dV/dsink relative-L2 <= 1e-2;
the bf16 case runs the d = 128 MFMA kernels (forward, both dK/dV schemes),
the float32 cases the generic kernels."""
import json
import math
import os
import sys

import numpy as np
import pytest
import torch

import ops_amd

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
with open(os.path.join(GOLDEN, "MANIFEST.json")) as f:
    MANIFEST = json.load(f)


def _case(name):
    z = np.load(os.path.join(GOLDEN, MANIFEST["file"]))
    return {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}


def _rel_l2(a, b):
    a, b = a.double(), torch.as_tensor(b).double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("name", sorted(MANIFEST["cases"]))
def test_hip_path_matches_golden(name):
    print(f"\n[gpu] golden fixture {name}", flush=True)
    sys.stdout.flush()
    c = MANIFEST["cases"][name]
    x = _case(name)
    dt = torch.bfloat16 if c["bf16"] else torch.float32
    q, k, v, dout = (torch.from_numpy(x[n]).to("cuda", dt) for n in ("q", "k", "v", "dout"))
    idx = torch.from_numpy(x["idx"]).cuda()
    kv_lens = torch.from_numpy(x["kv_lens"]).cuda() if "kv_lens" in x else None
    sink = torch.from_numpy(x["sink"]).cuda() if "sink" in x else None
    scale = float(x["scale"])
    out, lse = ops_amd.sfa_forward(q, k, v, idx, scale, kv_lens=kv_lens, attn_sink=sink)
    lse_c = lse.cpu().double()
    ref_l = torch.from_numpy(x["lse"])
    fin = torch.isfinite(ref_l)
    assert torch.equal(torch.isfinite(lse_c), fin)
    assert float((out.cpu().double() - torch.from_numpy(x["out"])).abs().max()) <= 2e-2
    assert float((lse_c[fin] - ref_l[fin]).abs().max()) <= 1e-3
    modes = ("csr", "atomic") if c["bf16"] else ("auto",)
    for mode in modes:
        dq, dk, dv, ds = ops_amd.sfa_backward(q, k, v, idx, out, lse, dout, scale, kv_lens=kv_lens, attn_sink=sink,
                                              dkv_mode=mode)
        for n, a in (("dq", dq), ("dk", dk), ("dv", dv)) + ((("dsink", ds),) if sink is not None else ()):
            e = _rel_l2(a.cpu(), x[n])
            assert e <= 1e-2, (mode, n, e)
