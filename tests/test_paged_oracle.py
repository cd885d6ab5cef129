"""The paged-KV mapping of the oracle (``paged_to_contiguous``) pinned without
restating it: a pure-Python loop over pages and rows on tiny inputs, the
identity page table (the pool is the cache), the round trip through
``ops_amd.workloads.page_kv`` (a seeded page shuffle with spare pages), and
planted mistakes (a swapped block-table entry, a lost unmapped-page rule)
that the loop comparison must catch.  Host checks of ``sfa_forward_paged``
need no GPU."""
import random

import pytest
import torch

import ops_amd
from ops_amd.workloads import make_workload, page_kv
from oracle.sfa_oracle import paged_to_contiguous, sfa_forward


def _loop_reference(k_cache, block_table, idx):
    """Row by row: logical key i of sequence b is row i % P of page bt[b][i // P]."""
    num_pages, P = k_cache.shape[:2]
    B, max_pages = block_table.shape
    k = torch.zeros(B, max_pages * P, *k_cache.shape[2:], dtype=k_cache.dtype)
    for b in range(B):
        for i in range(max_pages * P):
            pg = int(block_table[b, i // P])
            if 0 <= pg < num_pages:
                k[b, i] = k_cache[pg, i % P]
    out = idx.clone()
    for b in range(B):
        for t in range(idx.shape[1]):
            for g in range(idx.shape[2]):
                for j in range(idx.shape[3]):
                    i = int(idx[b, t, g, j])
                    if 0 <= i < max_pages * P:
                        pg = int(block_table[b, i // P])
                        if not 0 <= pg < num_pages:
                            out[b, t, g, j] = -1
    return k, out


def _tiny_case(seed):
    rng = random.Random(seed)
    torch.manual_seed(seed)
    num_pages, P, Hkv, D, B, max_pages = 7, 4, 2, 3, 3, 4
    k_cache = torch.randn(num_pages, P, Hkv, D, dtype=torch.float64)
    bt = torch.tensor([[rng.choice([-1, 9, 0, 1, 2, 3, 4, 5, 6]) for _ in range(max_pages)] for _ in range(B)],
                      dtype=torch.int32)
    idx = torch.tensor([rng.randrange(-3, max_pages * P + 3) for _ in range(B * 2 * Hkv * 6)],
                       dtype=torch.int32).view(B, 2, Hkv, 6)
    return k_cache, bt, idx


@pytest.mark.parametrize("seed", range(4))
def test_mapping_matches_loop(seed):
    k_cache, bt, idx = _tiny_case(seed)
    k, v, i2 = paged_to_contiguous(k_cache, k_cache[..., :2], bt, idx)
    k_ref, i_ref = _loop_reference(k_cache, bt, idx)
    assert torch.equal(k, k_ref)
    assert torch.equal(v, k_ref[..., :2])
    assert torch.equal(i2, i_ref)


def test_identity_table_is_a_reshape():
    torch.manual_seed(0)
    cache = torch.randn(2, 16, 1, 5)
    pool = cache.reshape(8, 4, 1, 5)
    bt = torch.arange(8, dtype=torch.int32).view(2, 4)
    idx = torch.randint(-1, 16, (2, 3, 1, 5), dtype=torch.int32)
    k, _, i2 = paged_to_contiguous(pool, pool, bt, idx)
    assert torch.equal(k, cache) and torch.equal(i2, idx)


@pytest.mark.parametrize("name,kw,page", [
    ("mla_decode", dict(B=3, Skv=512, K=64, Hq=4, ctx_lo=100), 64),
    ("train_gqa", dict(B=1, S=128, Hq=4, Hkv=2, K=32), 16),
])
def test_page_kv_round_trip(name, kw, page):
    w = make_workload(name, **kw)
    kp, vp, bt = page_kv(w.k, w.v, page, seed=3, spare_pages=5)
    assert kp.shape[0] == bt.numel() + 5
    k, v, idx = paged_to_contiguous(kp, vp, bt, w.idx)
    assert torch.equal(k, w.k) and torch.equal(v, w.v) and torch.equal(idx, w.idx)
    # the forward over the mapped cache is the forward over the original one
    o1, l1 = sfa_forward(w.q.float(), k.float(), v.float(), idx, w.scale, w.kv_lens)
    o2, l2 = sfa_forward(w.q.float(), w.k.float(), w.v.float(), w.idx, w.scale, w.kv_lens)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def _planted_transposed(k_cache, bt):
    """Wrong: row i // P of page bt[b][i % P] (page and row roles swapped)."""
    num_pages, P = k_cache.shape[:2]
    B, max_pages = bt.shape
    k = torch.zeros(B, max_pages * P, *k_cache.shape[2:], dtype=k_cache.dtype)
    for b in range(B):
        for i in range(max_pages * P):
            pg, r = int(bt[b, i % max_pages]), (i // max_pages) % P
            if 0 <= pg < num_pages:
                k[b, i] = k_cache[pg, r]
    return k


def test_planted_mistakes_are_caught():
    k_cache, bt, idx = _tiny_case(1)
    bt = bt.clone()
    bt[0, 0], bt[0, 1] = 2, 3
    k_ref, i_ref = _loop_reference(k_cache, bt, idx)
    swapped = bt.clone()
    swapped[0, 0], swapped[0, 1] = 3, 2
    assert not torch.equal(paged_to_contiguous(k_cache, k_cache, swapped, idx)[0], k_ref)
    assert not torch.equal(_planted_transposed(k_cache, bt), k_ref)
    # dropping the unmapped-page rule would keep every slot: the loop drops some
    k_cache, bt, idx = _tiny_case(2)
    _, i_ref = _loop_reference(k_cache, bt, idx)
    assert not torch.equal(idx, i_ref)
    assert torch.equal(paged_to_contiguous(k_cache, k_cache, bt, idx)[2], i_ref)


def test_paged_host_validation():
    q = torch.randn(1, 2, 4, 8)
    kc = torch.randn(6, 3, 1, 8)
    bt = torch.zeros(1, 2, dtype=torch.int32)
    idx = torch.zeros(1, 2, 1, 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="power of two"):
        ops_amd.sfa_forward_paged(q, kc, kc, bt, idx)
    kc = torch.randn(6, 4, 1, 8)
    with pytest.raises(ValueError, match="block_table"):
        ops_amd.sfa_forward_paged(q, kc, kc, bt[0], idx)
    with pytest.raises(ValueError, match="GPU"):
        ops_amd.sfa_forward_paged(q, kc, kc, bt, idx)
