"""GPU test of sfa_fwd_noalloc, the forward entry point that allocates
nothing (split-k partials and the persistent prefill's claim counters in the
library's static per-GPU scratch), called through the C ABI: its results
must be bitwise those of sfa_fwd (same kernels, same split plan, caller
workspace) and within the oracle's bars, on two calls in a row, the second
with a smaller input (a different kernel family), and again on the first
input afterwards."""
import ctypes
import math
import sys

import pytest
import torch

from ops_amd import _lib
from ops_amd import sfa as sfa_mod
from ops_amd.workloads import make_workload
from oracle.sfa_oracle import sfa_forward as ref_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(f"\n[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _decode_case(B, Skv, Hq, Hkv, Dqk, Dv, K, seed, shared_kv):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, 1, Hq, Dqk, generator=g).bfloat16()
    k = torch.randn(B, Skv, Hkv, Dqk, generator=g).bfloat16()
    v = k[..., :Dv] if shared_kv else torch.randn(B, Skv, Hkv, Dv, generator=g).bfloat16()
    kv_lens = torch.randint(Skv // 2, Skv + 1, (B,), generator=g, dtype=torch.int32)
    idx = torch.full((B, 1, Hkv, K), -1, dtype=torch.int32)
    for b in range(B):
        for h in range(Hkv):
            n = min(K, int(kv_lens[b]))
            idx[b, 0, h, :n] = torch.randperm(int(kv_lens[b]), generator=g)[:n].to(torch.int32)
    return q, k, v, idx, kv_lens


def _run(entry, q, k, v, idx, kv_lens, scale, idx_sorted=False):
    """One call of sfa_fwd (caller workspace) or sfa_fwd_noalloc through the
    C ABI on torch's current stream; returns (out, lse, workspace bytes)."""
    lib = _lib.load()
    B, Sq, Hq, _ = q.shape
    out = torch.empty(B, Sq, Hq, v.shape[3], dtype=q.dtype, device=DEV)
    lse = torch.empty(B, Sq, Hq, dtype=torch.float32, device=DEV)
    a = sfa_mod._fwd_args(q, k, v, idx, out, lse, scale, kv_lens, None, 0, idx_sorted)
    ws = lib.sfa_fwd_workspace_size(ctypes.byref(a))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if entry == "noalloc":
        rc = lib.sfa_fwd_noalloc(ctypes.byref(a), stream)
    else:
        wbuf = torch.empty(ws, dtype=torch.uint8, device=DEV)
        rc = lib.sfa_fwd(ctypes.byref(a), ctypes.c_void_p(wbuf.data_ptr()), ws, stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return out, lse, ws


def _check_oracle(out, lse, q, k, v, idx, kv_lens, scale):
    o_ref, l_ref = ref_forward(q, k, v, idx, scale, kv_lens=kv_lens)
    err_o = float((out.float().cpu() - o_ref).abs().max())
    err_l = float((lse.cpu() - l_ref).abs().max())
    assert err_o <= 2e-2 and err_l <= 1e-3, (err_o, err_l)


def test_noalloc_matches_sfa_fwd_on_consecutive_calls():
    cases = [
        # MLA decode shape: 16 sequences x 128 heads, 16 splits (33.6 MB of partials)
        ("mla B=16 Skv=8192 Hq=128 d 576/512 K=2048", dict(B=16, Skv=8192, Hq=128, Hkv=1, Dqk=576, Dv=512, K=2048,
                                                          seed=1, shared_kv=True)),
        # smaller: d=128 GQA decode, 2 sequences x 2 kv heads, 8 splits (the d=128 kernel)
        ("d128 B=2 Skv=1024 Hq=32 Hkv=2 K=256", dict(B=2, Skv=1024, Hq=32, Hkv=2, Dqk=128, Dv=128, K=256, seed=2,
                                                     shared_kv=False)),
    ]
    cases.append(cases[0])  # the first input again, after the smaller call
    sizes = []
    for name, c in cases:
        _say(f"sfa_fwd_noalloc vs sfa_fwd: {name}")
        q, k, v, idx, kv_lens = _decode_case(**c)
        scale = 1.0 / math.sqrt(c["Dqk"])
        dq, dk, dv, di, dl = (t.to(DEV) for t in (q, k, v, idx, kv_lens))
        if c["shared_kv"]:
            dv = dk[..., :c["Dv"]]
        o_na, l_na, ws = _run("noalloc", dq, dk, dv, di, dl, scale)
        o_ws, l_ws, _ = _run("workspace", dq, dk, dv, di, dl, scale)
        assert 0 < ws <= _lib.SFA_NOALLOC_SCRATCH_BYTES
        sizes.append(ws)
        assert torch.equal(o_na, o_ws) and torch.equal(l_na, l_ws), name
        _check_oracle(o_na, l_na, q.float(), k.float(), v.float(), idx, kv_lens, scale)
    assert sizes[1] < sizes[0]


def test_noalloc_persistent_prefill_after_decode():
    """MLA prefill at S = 4100 (>= 4096 items: the persistent schedule, whose
    per-XCD claim counters sit in the static scratch and are cleared by a fill
    kernel on every call) right after a decode call that left split-k partials
    there, then a smaller prefill (S = 1000, plain grid): bitwise equal to
    sfa_fwd, sampled rows within the oracle's bars."""
    dec = dict(B=2, Skv=1024, Hq=32, Hkv=2, Dqk=128, Dv=128, K=256, seed=3, shared_kv=False)
    q, k, v, idx, kv_lens = (t.to(DEV) for t in _decode_case(**dec))
    _run("noalloc", q, k, v, idx, kv_lens, 1.0 / math.sqrt(128))
    sizes = []
    for S in (4100, 1000):
        _say(f"sfa_fwd_noalloc vs sfa_fwd: mla prefill S={S} K=256 Hq=128")
        w = make_workload("mla_prefill", device=DEV, S=S, K=256)
        o_na, l_na, ws = _run("noalloc", w.q, w.k, w.v, w.idx, None, w.scale)
        o_ws, l_ws, _ = _run("workspace", w.q, w.k, w.v, w.idx, None, w.scale)
        sizes.append(ws)
        assert ws <= _lib.SFA_NOALLOC_SCRATCH_BYTES
        assert torch.equal(o_na, o_ws) and torch.equal(l_na, l_ws), S
        rows = torch.tensor([0, 1, 255, 256, S // 2, S - 2, S - 1])
        o_ref, l_ref = ref_forward(w.q[:, rows].float().cpu(), w.k.float().cpu(), w.v.float().cpu(),
                                   w.idx[:, rows].cpu(), w.scale)
        err_o = float((o_na[:, rows].float().cpu() - o_ref).abs().max())
        err_l = float((l_na[:, rows].cpu() - l_ref).abs().max())
        assert err_o <= 2e-2 and err_l <= 1e-3, (S, err_o, err_l)
    assert sizes[0] > 0 and sizes[1] == 0


def test_noalloc_prefill_rows_beyond_the_scratch_walk_their_own_order():
    """MLA prefill at S = 8192, top-k 2048: its index rows in ascending order
    (64 MiB) and the claim counters do not fit the static scratch together,
    so sfa_fwd_noalloc skips the sort pass and walks the caller's rows in
    their own order: bitwise sfa_fwd with SFA_FWD_IDX_SORTED set (no pass),
    sampled rows within the oracle's bars."""
    S, K = 8192, 2048
    _say(f"sfa_fwd_noalloc vs sfa_fwd (rows declared sorted): mla prefill S={S} K={K} Hq=128")
    w = make_workload("mla_prefill", device=DEV, S=S, K=K)
    lib = _lib.load()
    out = torch.empty(1, S, 128, 512, dtype=w.q.dtype, device=DEV)
    lse = torch.empty(1, S, 128, dtype=torch.float32, device=DEV)
    a = sfa_mod._fwd_args(w.q, w.k, w.v, w.idx, out, lse, w.scale, None, None, 0)
    assert lib.sfa_fwd_workspace_size(ctypes.byref(a)) > _lib.SFA_NOALLOC_SCRATCH_BYTES
    o_na, l_na, _ = _run("noalloc", w.q, w.k, w.v, w.idx, None, w.scale)
    o_ws, l_ws, ws = _run("workspace", w.q, w.k, w.v, w.idx, None, w.scale, idx_sorted=True)
    assert 0 < ws <= _lib.SFA_NOALLOC_SCRATCH_BYTES
    assert torch.equal(o_na, o_ws) and torch.equal(l_na, l_ws)
    rows = torch.tensor([0, 1, 2047, 2048, S // 2, S - 1])
    o_ref, l_ref = ref_forward(w.q[:, rows].float().cpu(), w.k.float().cpu(), w.v.float().cpu(),
                               w.idx[:, rows].cpu(), w.scale)
    err_o = float((o_na[:, rows].float().cpu() - o_ref).abs().max())
    err_l = float((l_na[:, rows].cpu() - l_ref).abs().max())
    assert err_o <= 2e-2 and err_l <= 1e-3, (err_o, err_l)
