"""GPU parity of the MLA shared-KV backward at the sizes the benchmark times
and at shapes that reach its multi-word index maps and chunk boundaries.

* The full MLA prefill workload (B=1, S=32768, Hq=128, d_qk 576 / d_v 512,
  top-k 2048) in both dK/dV modes: 32 chunks of 1024 queries, 1024 bitmap
  words per query and a reduction over 32768 keys in the deterministic mode.
  Gradients are written into NaN-filled tensors, so every row must be
  written; dQ of sampled query rows is checked against the CPU oracle and the
  shared-row gradient dK + dV of sampled keys (early keys that thousands of
  queries select, recency-window keys, the last keys, unreferenced keys)
  against the float32 per-key evaluation of tests/fullgrid_ref.py (pinned to
  the oracle by tests/test_fullgrid_ref.py).
* Skv = 8192 with two sequences, a sink, a gradient on LSE, kv_lens, a fully
  masked query row and out-of-range ids: every row against the float32
  full-grid evaluation.
* Two sequences and two KV heads (Hq = 256, G = 128) sized so that chunk
  boundaries fall inside a sequence in both modes.

Bars: relative L2 <= 1e-2 (SFA.py:849-853 sums dK and dV of the shared rows
into one buffer; so does this path), per-row relative error <= 5e-2, exact
zeros for unreferenced rows."""
import math
import sys

import pytest
import torch

import fullgrid_ref as fr
import ops_amd
from ops_amd.workloads import make_workload
from oracle.sfa_oracle import sfa_backward as ref_backward

pytestmark = pytest.mark.gpu

DEV = "cuda"
GRAD_RL2, ROW_TOL = 1e-2, 5e-2


def _say(msg):
    print(f"\n[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _rel_l2(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _bwd_nan(q, kv, idx, out, lse, dout, scale, mode, **kw):
    """sfa_backward (C ABI, merged shared rows) into NaN-filled dq / dkv."""
    dq = torch.full(q.shape, float("nan"), dtype=q.dtype, device=DEV)
    dkv = torch.full(kv.shape, float("nan"), dtype=kv.dtype, device=DEV)
    ops_amd.sfa_backward(q, kv, kv[..., :512], idx, out, lse, dout, scale, merge_kv=True, dkv_mode=mode,
                         dq=dq, dk=dkv, **kw)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(dq).all()), "unwritten or non-finite dQ rows"
    assert bool(torch.isfinite(dkv).all()), "unwritten or non-finite dK + dV rows"
    return dq, dkv


def _merged(dk, dv):
    m = dk.clone()
    m[..., :dv.shape[-1]] += dv
    return m


@pytest.fixture(scope="module")
def full_mla():
    _say("full MLA prefill workload: S=32768 Hq=128 K=2048 (forward on the GPU)")
    w = make_workload("mla_prefill", device=DEV, with_dout=True)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    torch.cuda.synchronize()
    return w, out, lse


@pytest.mark.parametrize("mode", ["auto", "atomic"])
def test_mla_bwd_full_workload(full_mla, mode):
    w, out, lse = full_mla
    S = w.q.shape[1]
    _say(f"MLA bwd at the full workload, dkv_mode={mode}: every row written, sampled rows vs the oracle")
    dq, dkv = _bwd_nan(w.q, w.k, w.idx, out, lse, w.dout, w.scale, mode)

    # dQ of sampled queries: the CPU oracle on those rows (dQ of a query
    # depends only on its own row, the keys and the forward's out / lse)
    g = torch.Generator().manual_seed(5)
    rows = torch.cat([torch.tensor([0, 1, 2047, 2048, 2049, 16383, S - 2, S - 1]),
                      torch.randint(0, S, (8,), generator=g)])
    rq, _, _, _ = ref_backward(w.q[:, rows].float().cpu(), w.k.float().cpu(), w.v.float().cpu(),
                               w.idx[:, rows].cpu(), out[:, rows].float().cpu(), lse[:, rows].cpu(),
                               w.dout[:, rows].float().cpu(), w.scale)
    got = dq[:, rows].float().cpu()
    e_q, er_q = _rel_l2(got, rq), fr.rowwise_rel_err(got, rq)
    _say(f"  dQ on {rows.numel()} rows: rel-L2 {e_q:.2e}, worst row {er_q:.2e}")
    assert e_q <= GRAD_RL2 and er_q <= ROW_TOL

    # dK + dV of sampled keys, from the (query, slot) pairs that select them
    iv = w.idx[0, :, 0]
    cnt = torch.bincount(iv[iv >= 0].long(), minlength=S)
    unref = (cnt == 0).nonzero().flatten()
    hot = torch.topk(cnt.float(), 3).indices
    keys = [0, 1, 7, 1000, 2047, 16384, 31000, 32000] + hot.tolist() + [S - 2, S - 1]
    _say(f"  keys {keys}: references {[int(cnt[j]) for j in keys]}; {unref.numel()} unreferenced keys")
    rk, rv = fr.key_grads(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale, keys)
    ref = _merged(rk, rv)
    got = dkv[0, keys, 0].float()
    e_kv, er_kv = _rel_l2(got, ref), fr.rowwise_rel_err(got, ref)
    _say(f"  dK + dV on {len(keys)} keys: rel-L2 {e_kv:.2e}, worst row {er_kv:.2e}")
    assert e_kv <= GRAD_RL2 and er_kv <= ROW_TOL
    if unref.numel():
        assert bool((dkv[0, unref] == 0).all()), "unreferenced keys get exactly zero"


@pytest.mark.parametrize("mode", ["auto", "atomic"])
def test_mla_bwd_skv8192_masking_sink_dlse(mode):
    """Skv = 8192 (256 bitmap words per query, 16 chunks of 1024 queries over
    both sequences in the deterministic mode) with interior and trailing padding, ids past Skv and
    past kv_lens, a fully masked row, a sink and a gradient on LSE."""
    _say(f"MLA bwd B=2 S=8192 Hq=128 K=2048 sink/dlse/kv_lens/masked row, dkv_mode={mode}")
    w = make_workload("mla_prefill", device=DEV, seed=2, B=2, S=8192, with_dout=True)
    B, S = 2, 8192
    gen = torch.Generator(device=DEV).manual_seed(17)
    idx = w.idx.clone()
    drop = torch.rand(idx.shape, device=DEV, generator=gen) < 0.05
    idx = torch.where(drop, torch.full_like(idx, -1), idx)          # interior -1
    idx[0, 100] = -1                                                 # a fully masked query
    idx[1, 5000, 0, :7] = S + 11                                     # ids past Skv
    kv_lens = torch.tensor([S, 6000], device=DEV, dtype=torch.int32)  # ids >= 6000 invalid in batch 1
    sink = torch.randn(128, device=DEV, generator=gen)
    dlse = torch.randn(B, S, 128, device=DEV, generator=gen)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, idx, w.scale, kv_lens=kv_lens, attn_sink=sink)
    dq = torch.full(w.q.shape, float("nan"), dtype=w.q.dtype, device=DEV)
    dkv = torch.full(w.k.shape, float("nan"), dtype=w.k.dtype, device=DEV)
    _, _, _, dsink = ops_amd.sfa_backward(w.q, w.k, w.v, idx, out, lse, w.dout, w.scale, kv_lens=kv_lens,
                                          attn_sink=sink, dlse=dlse, merge_kv=True, dkv_mode=mode, dq=dq, dk=dkv)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(dq).all()) and bool(torch.isfinite(dkv).all())
    rq, rk, rv, rs = fr.backward(w.q, w.k, w.v, idx, out, lse, w.dout, w.scale, kv_lens=kv_lens, sink=sink,
                                 dlse=dlse)
    rkv = _merged(rk, rv)
    for nm, a, r in (("dq", dq, rq), ("dkv", dkv, rkv)):
        e, er = _rel_l2(a.float(), r), fr.rowwise_rel_err(a, r)
        _say(f"  {nm}: rel-L2 {e:.2e}, worst row {er:.2e}")
        assert e <= GRAD_RL2 and er <= ROW_TOL, (nm, e, er)
    e_s = _rel_l2(dsink, rs)
    _say(f"  dsink: rel-L2 {e_s:.2e}")
    assert e_s <= GRAD_RL2
    assert bool((dq[0, 100] == 0).all()), "a query with no valid slot has dQ = 0"
    assert bool((dkv[1, 6000:] == 0).all()), "rows past kv_lens get no gradient"
    unref = rkv.abs().amax(-1) == 0
    assert bool((dkv[unref] == 0).all())


def _causal_rows(B, S, Hkv, K, gen):
    """Per (batch, kv head, query) a random subset of min(K, t + 1) keys of
    [0, t] in random order, -1 padded (different rows for each kv head)."""
    idx = torch.full((B, S, Hkv, K), -1, dtype=torch.int32)
    for b in range(B):
        for g in range(Hkv):
            u = torch.rand(S, S, generator=gen)
            u = torch.where(torch.ones(S, S, dtype=torch.bool).tril(), u, torch.full_like(u, -1.0))
            order = torch.argsort(u, dim=1, descending=True)[:, :min(K, S)]
            n = torch.clamp(torch.arange(S) + 1, max=K)
            keep = torch.arange(order.shape[1])[None, :] < n[:, None]
            idx[b, :, g, :order.shape[1]] = torch.where(keep, order, torch.full_like(order, -1)).to(torch.int32)
    return idx


@pytest.mark.parametrize("mode", ["auto", "atomic"])
def test_mla_bwd_two_kv_heads_chunk_inside_sequence(mode):
    """B = 2, Hq = 256 over Hkv = 2 (G = 128), S = 640, top-k 2048: 2560 work
    items, so the deterministic mode's 1024-item chunks and the atomic mode's
    2048-item chunk both end inside a sequence, and the reduction's item range
    per (batch, kv head) starts mid-sequence with a stride of two kv heads."""
    _say(f"MLA bwd B=2 S=640 Hq=256 Hkv=2 K=2048, dkv_mode={mode}")
    B, S, Hq, Hkv, K = 2, 640, 256, 2, 2048
    gen = torch.Generator().manual_seed(23)
    q = torch.randn(B, S, Hq, 576, generator=gen).bfloat16().to(DEV)
    kv = torch.randn(B, S, Hkv, 576, generator=gen).bfloat16().to(DEV)
    dout = torch.randn(B, S, Hq, 512, generator=gen).bfloat16().to(DEV)
    idx = _causal_rows(B, S, Hkv, K, gen).to(DEV)
    scale = 1.0 / math.sqrt(576)
    out, lse = ops_amd.sfa_forward(q, kv, kv[..., :512], idx, scale)
    dq, dkv = _bwd_nan(q, kv, idx, out, lse, dout, scale, mode)
    rq, rk, rv, _ = fr.backward(q, kv, kv[..., :512], idx, out, lse, dout, scale)
    rkv = _merged(rk, rv)
    for nm, a, r in (("dq", dq, rq), ("dkv", dkv, rkv)):
        e, er = _rel_l2(a.float(), r), fr.rowwise_rel_err(a, r)
        _say(f"  {nm}: rel-L2 {e:.2e}, worst row {er:.2e}")
        assert e <= GRAD_RL2 and er <= ROW_TOL, (nm, e, er)
