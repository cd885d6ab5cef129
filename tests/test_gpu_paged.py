"""GPU parity of the paged-KV forward (``sfa_fwd_paged`` through the C ABI).

The same kernels serve both layouts; only the index staging (block-table
translation) and the row addresses differ, so the paged result must be
bitwise identical to the contiguous forward on the cache the block table
describes, for every kernel family (MLA, d = 128, generic fp32), split count,
sink and kv_lens.  Each case is also held to the oracle bars (O max-abs
<= 2e-2, LSE <= 1e-3) through ``paged_to_contiguous``.  Unmapped pages make
their slots invalid; a full-size decode cache paged into a 4.8 GB pool
exercises row addresses beyond 4 GiB."""
import math
import sys

import pytest
import torch

import ops_amd
from ops_amd.workloads import make_workload, page_kv
from oracle.sfa_oracle import paged_to_contiguous
from oracle.sfa_oracle import sfa_forward as ref_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"
O_TOL = 2e-2
LSE_TOL = 1e-3


def _say(msg):
    print(f"\n[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _check_oracle(out, lse, o_ref, l_ref):
    out, lse = out.float().cpu(), lse.float().cpu()
    fin = torch.isfinite(l_ref)
    assert torch.equal(torch.isfinite(lse), fin)
    assert float((out - o_ref).abs().max()) <= O_TOL
    if fin.any():
        assert float((lse[fin] - l_ref[fin]).abs().max()) <= LSE_TOL


CASES = [
    # (name, overrides, page_size, num_splits, with_sink): kernel family in the id
    ("mla_decode", dict(B=4, Skv=2048, K=512, ctx_lo=300), 64, 0, False),
    ("mla_decode", dict(B=3, Skv=1024, K=256, ctx_lo=100), 16, 3, True),
    ("mla_prefill", dict(S=256, K=128), 32, 0, True),
    ("prefill", dict(S=512, K=64), 16, 0, False),
    ("train_gqa", dict(B=1, S=512, K=128), 32, 2, True),
    ("tiny", dict(), 8, 0, True),
    ("prefill", dict(S=256, K=64, Hq=8, Dqk=64, Dv=64), 16, 2, True),
]


@pytest.mark.parametrize("name,kw,page,splits,with_sink", CASES,
                         ids=["mla-decode", "mla-decode-splits3-sink", "mla-prefill-sink", "d128-mqa",
                              "d128-gqa-splits2-sink", "generic-fp32-sink", "d64-mqa-splits2-sink"])
def test_paged_equals_contiguous(name, kw, page, splits, with_sink):
    _say(f"paged {name} {kw} page={page} splits={splits} sink={with_sink}")
    w = make_workload(name, device=DEV, **kw)
    Hq = w.q.shape[2]
    sink = torch.linspace(-1.0, 2.0, Hq, device=DEV) if with_sink else None
    kp, vp, bt = page_kv(w.k, w.v, page, seed=11, spare_pages=7)
    o_c, l_c = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, w.kv_lens, sink, num_splits=splits)
    o_p, l_p = ops_amd.sfa_forward_paged(w.q, kp, vp, bt, w.idx, w.scale, w.kv_lens, sink, num_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_c)
    assert torch.equal(l_p, l_c)
    k2, v2, i2 = paged_to_contiguous(kp.cpu(), vp.cpu(), bt.cpu(), w.idx.cpu())
    o_r, l_r = ref_forward(w.q.cpu().float(), k2.float(), v2.float(), i2, w.scale,
                           None if w.kv_lens is None else w.kv_lens.cpu(), None if sink is None else sink.cpu())
    _check_oracle(o_p, l_p, o_r, l_r)


@pytest.mark.parametrize("name,kw,page", [
    ("mla_decode", dict(B=4, Skv=2048, K=512, ctx_lo=1500), 64),
    ("prefill", dict(S=512, K=64), 16),
    ("tiny", dict(), 8),
], ids=["mla", "d128", "generic-fp32"])
def test_unmapped_pages_drop_their_slots(name, kw, page):
    _say(f"paged {name}: unmapped block-table entries")
    w = make_workload(name, device=DEV, **kw)
    kp, vp, bt = page_kv(w.k, w.v, page, seed=5)
    bt = bt.clone()
    g = torch.Generator(device="cpu")
    g.manual_seed(3)
    hole = torch.rand(bt.shape, generator=g) < 0.25
    junk = torch.where(torch.rand(bt.shape, generator=g) < 0.5, -1, kp.shape[0] + 3).to(torch.int32)
    bt = torch.where(hole.to(DEV), junk.to(DEV), bt)
    k2, v2, i2 = paged_to_contiguous(kp.cpu(), vp.cpu(), bt.cpu(), w.idx.cpu())
    assert not torch.equal(i2, w.idx.cpu()), "the holes must hit referenced pages"
    o_p, l_p = ops_amd.sfa_forward_paged(w.q, kp, vp, bt, w.idx, w.scale, w.kv_lens)
    # the contiguous forward of the original cache with the dropped slots set to -1
    o_c, l_c = ops_amd.sfa_forward(w.q, w.k, w.v, i2.to(DEV), w.scale, w.kv_lens)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_c)
    assert torch.equal(l_p, l_c)


def test_full_decode_pool_beyond_4gib():
    _say("paged mla_decode full size: B=64 Skv=65536 page 64, 4.8 GB pool")
    w = make_workload("mla_decode", device=DEV)
    kp, vp, bt = page_kv(w.k, w.v, 64, seed=2)
    assert kp.numel() * kp.element_size() > (1 << 32)
    # the shuffle must place referenced rows beyond 4 GiB of the pool
    rows = (bt.long()[:, :, None] * 64 + torch.arange(64, device=DEV)).view(64, -1)
    ref_rows = torch.gather(rows, 1, w.idx.view(64, -1).long().clamp_min(0))
    assert int(ref_rows.max()) * 576 * 2 > (1 << 32)
    o_c, l_c = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, w.kv_lens)
    o_p, l_p = ops_amd.sfa_forward_paged(w.q, kp, vp, bt, w.idx, w.scale, w.kv_lens)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_c)
    assert torch.equal(l_p, l_c)
    assert torch.isfinite(l_p).all()
    del kp, vp
    torch.cuda.empty_cache()


def test_single_row_pages_and_padded_table():
    # page_size 1 (shift 0) and a block table whose rows are longer than the
    # pages in use (row stride > max_pages)
    _say("paged mla_decode: page_size 1, padded block-table rows")
    w = make_workload("mla_decode", device=DEV, B=3, Skv=512, K=128, ctx_lo=200)
    kp, vp, bt = page_kv(w.k, w.v, 1, seed=4, spare_pages=9)
    wide = torch.full((bt.shape[0], bt.shape[1] + 37), -1, dtype=torch.int32, device=DEV)
    wide[:, :bt.shape[1]] = bt
    bt_view = wide[:, :bt.shape[1]]            # stride(0) = max_pages + 37
    assert bt_view.stride(0) > bt_view.shape[1]
    o_c, l_c = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, w.kv_lens)
    o_p, l_p = ops_amd.sfa_forward_paged(w.q, kp, vp, bt_view, w.idx, w.scale, w.kv_lens)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_c)
    assert torch.equal(l_p, l_c)



def test_paged_persistent_mla_prefill():
    """MLA prefill at S = 4160 (>= 4096 work items: the persistent kernel,
    which stages scaled pool offsets for its paged gathers) with 64-row
    pages shuffled over the pool and a sink: bitwise equal to the contiguous
    forward; sampled rows within the oracle's bars."""
    _say("paged mla_prefill persistent S=4160 K=256 page=64 sink")
    w = make_workload("mla_prefill", device=DEV, S=4160, K=256)
    Hq = w.q.shape[2]
    sink = torch.linspace(-1.0, 2.0, Hq, device=DEV)
    kp, vp, bt = page_kv(w.k, w.v, 64, seed=5, spare_pages=3)
    o_c, l_c = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, None, sink)
    o_p, l_p = ops_amd.sfa_forward_paged(w.q, kp, vp, bt, w.idx, w.scale, None, sink)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_c)
    assert torch.equal(l_p, l_c)
    rows = torch.tensor([0, 1, 255, 1000, 2047, 2048, 4095, 4159])
    k2, v2, i2 = paged_to_contiguous(kp.cpu(), vp.cpu(), bt.cpu(), w.idx[:, rows].cpu())
    o_r, l_r = ref_forward(w.q[:, rows].cpu().float(), k2.float(), v2.float(), i2, w.scale, None, sink.cpu())
    _check_oracle(o_p[:, rows], l_p[:, rows], o_r, l_r)


@pytest.mark.parametrize("G", [20, 64])
def test_paged_d128_large_groups(G):
    """d = 128 with more than 16 query heads on one kv head (the reference's
    shape class) over a paged pool: the paged forward runs the head-group
    kernel (one workgroup per 16 heads), the contiguous one the shared-tile
    kernel (the head groups as waves of one workgroup): both against the
    oracle (with a sink and kv_lens), and bitwise equal to each other, since
    a wave's arithmetic is the same in both kernels."""
    _say(f"paged d=128 G={G} S=256 K=96 page=16 sink")
    w = make_workload("prefill", device=DEV, S=256, Hq=G, K=96, seed=7)
    sink = torch.linspace(-1.0, 2.0, G, device=DEV)
    kv_lens = torch.tensor([200], dtype=torch.int32, device=DEV)
    kp, vp, bt = page_kv(w.k, w.v, 16, seed=13, spare_pages=5)
    o_c, l_c = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, kv_lens, sink)
    o_p, l_p = ops_amd.sfa_forward_paged(w.q, kp, vp, bt, w.idx, w.scale, kv_lens, sink)
    torch.cuda.synchronize()
    k2, v2, i2 = paged_to_contiguous(kp.cpu(), vp.cpu(), bt.cpu(), w.idx.cpu())
    o_r, l_r = ref_forward(w.q.cpu().float(), k2.float(), v2.float(), i2, w.scale, kv_lens.cpu(), sink.cpu())
    _check_oracle(o_p, l_p, o_r, l_r)
    _check_oracle(o_c, l_c, o_r, l_r)
    assert torch.equal(o_p, o_c) and torch.equal(l_p, l_c)
