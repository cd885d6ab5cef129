"""Pins the CPU oracle (oracle/sfa_oracle.py) against checks that do not
restate its formulas: a pure-Python fp64 loop brute force, torch's
scaled_dot_product_attention on the dense causal special case, autograd /
gradcheck, closed forms and exact index invariants.  The reference
(SFA.py) ships no tests or golden vectors, so these are the pins."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle.sfa_oracle import (count_valid_pairs, sfa_backward, sfa_forward, sfa_forward_autograd,
                               valid_mask)


def _rand_case(B=1, S=10, Skv=None, Hq=4, Hkv=2, Dqk=8, Dv=6, K=5, seed=0, dtype=torch.float64, pad=True):
    g = torch.Generator().manual_seed(seed)
    Skv = Skv or S
    q = torch.randn(B, S, Hq, Dqk, generator=g, dtype=dtype)
    k = torch.randn(B, Skv, Hkv, Dqk, generator=g, dtype=dtype)
    v = torch.randn(B, Skv, Hkv, Dv, generator=g, dtype=dtype)
    idx = torch.randint(0, Skv, (B, S, Hkv, K), generator=g, dtype=torch.int32)
    if pad:
        # -1 anywhere (interior too), some out-of-range values, keep >= 1 valid per row
        r = torch.rand(B, S, Hkv, K, generator=g)
        idx = torch.where(r < 0.2, torch.full_like(idx, -1), idx)
        idx = torch.where((r >= 0.2) & (r < 0.27), torch.full_like(idx, Skv + 3), idx)
        idx[..., 0] = torch.randint(0, Skv, (B, S, Hkv), generator=g, dtype=torch.int32)
    do = torch.randn(B, S, Hq, Dv, generator=g, dtype=dtype)
    return q, k, v, idx, do


def _brute_forward(q, k, v, idx, scale, kv_lens=None, sink=None):
    """Pure-Python fp64 loops over every (b, t, h, slot)."""
    B, S, Hq, Dqk = q.shape
    Skv, Hkv, Dv = k.shape[1], k.shape[2], v.shape[3]
    G = Hq // Hkv
    out = [[[[0.0] * Dv for _ in range(Hq)] for _ in range(S)] for _ in range(B)]
    lse = [[[0.0] * Hq for _ in range(S)] for _ in range(B)]
    Q, Kt, V, I = q.tolist(), k.tolist(), v.tolist(), idx.tolist()
    for b in range(B):
        bound = Skv if kv_lens is None else min(int(kv_lens[b]), Skv)
        for t in range(S):
            for h in range(Hq):
                g = h // G
                scores, rows = [], []
                for j in I[b][t][g]:
                    if 0 <= j < bound:
                        scores.append(scale * sum(a * c for a, c in zip(Q[b][t][h], Kt[b][j][g])))
                        rows.append(j)
                terms = list(scores) + ([float(sink[h])] if sink is not None else [])
                if not terms:
                    lse[b][t][h] = -math.inf
                    continue
                m = max(terms)
                z = sum(math.exp(x - m) for x in terms)
                L = m + math.log(z)
                lse[b][t][h] = L
                for s_, j in zip(scores, rows):
                    w = math.exp(s_ - L)
                    for d in range(Dv):
                        out[b][t][h][d] += w * V[b][j][g][d]
    return torch.tensor(out, dtype=torch.float64), torch.tensor(lse, dtype=torch.float64)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_forward_matches_brute_force(seed):
    q, k, v, idx, _ = _rand_case(seed=seed)
    o, l = sfa_forward(q, k, v, idx, scale=0.37, dtype=torch.float64)
    ob, lb = _brute_forward(q, k, v, idx, 0.37)
    torch.testing.assert_close(o, ob, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(l, lb, rtol=1e-12, atol=1e-12)


def test_forward_kv_lens_and_sink_match_brute_force():
    q, k, v, idx, _ = _rand_case(B=2, S=7, Skv=9, seed=5)
    kv_lens = torch.tensor([4, 9], dtype=torch.int32)
    sink = torch.tensor([0.3, -1.0, 2.0, 0.0], dtype=torch.float64)
    o, l = sfa_forward(q, k, v, idx, scale=0.5, kv_lens=kv_lens, sink=sink, dtype=torch.float64)
    ob, lb = _brute_forward(q, k, v, idx, 0.5, kv_lens=kv_lens, sink=sink)
    torch.testing.assert_close(o, ob, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(l, lb, rtol=1e-12, atol=1e-12)


def test_dense_causal_matches_sdpa():
    """idx row t = all of [0, t] in random order: SFA == causal dense attention
    (torch's library SDPA, GQA heads repeated)."""
    B, S, Hq, Hkv, D = 2, 16, 4, 2, 8
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, S, Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, S, Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, S, Hkv, D, generator=g, dtype=torch.float64)
    idx = torch.full((B, S, Hkv, S), -1, dtype=torch.int32)
    for b in range(B):
        for h in range(Hkv):
            for t in range(S):
                perm = torch.randperm(t + 1, generator=g)
                idx[b, t, h, :t + 1] = perm.to(torch.int32)
    o, l = sfa_forward(q, k, v, idx, dtype=torch.float64)
    G = Hq // Hkv
    kr = k.repeat_interleave(G, dim=2).transpose(1, 2)
    vr = v.repeat_interleave(G, dim=2).transpose(1, 2)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), kr, vr, is_causal=True).transpose(1, 2)
    torch.testing.assert_close(o, ref, rtol=1e-10, atol=1e-10)
    scores = torch.einsum("bshd,bthd->bhst", q.transpose(1, 2).transpose(1, 2), kr.transpose(1, 2)) / math.sqrt(D)
    mask = torch.ones(S, S, dtype=torch.bool).tril()
    lse_ref = torch.logsumexp(scores.masked_fill(~mask, -math.inf), dim=-1).transpose(1, 2)
    torch.testing.assert_close(l, lse_ref, rtol=1e-10, atol=1e-10)


def test_explicit_backward_matches_autograd():
    q, k, v, idx, do = _rand_case(B=2, S=6, Hq=4, Hkv=2, seed=7)
    sink = torch.tensor([0.1, -0.5, 1.5, 0.2], dtype=torch.float64)
    kv_lens = torch.tensor([5, 6], dtype=torch.int32)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, sink)]
    o, l = sfa_forward_autograd(leaves[0], leaves[1], leaves[2], idx, scale=0.4, kv_lens=kv_lens, sink=leaves[3])
    dl = torch.randn(l.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    (o * do).sum().backward()
    dq, dk, dv, ds = sfa_backward(q, k, v, idx, o.detach(), l.detach(), do, scale=0.4, kv_lens=kv_lens, sink=sink,
                                  dtype=torch.float64)
    torch.testing.assert_close(dq, leaves[0].grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dk, leaves[1].grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dv, leaves[2].grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(ds, leaves[3].grad, rtol=1e-10, atol=1e-10)
    del dl


def test_gradcheck_fp64():
    q, k, v, idx, _ = _rand_case(B=1, S=5, Hq=4, Hkv=2, Dqk=4, Dv=3, K=4, seed=11)
    inputs = tuple(x.clone().requires_grad_(True) for x in (q, k, v))

    def f(q_, k_, v_):
        o, l = sfa_forward_autograd(q_, k_, v_, idx, scale=0.6)
        return o, l

    assert torch.autograd.gradcheck(f, inputs, eps=1e-6, atol=1e-7)


def test_closed_form_single_index():
    q, k, v, idx, _ = _rand_case(B=1, S=4, Hq=2, Hkv=1, K=3, seed=2, pad=False)
    idx[..., :] = -1
    idx[0, :, 0, 1] = torch.tensor([3, 0, 2, 1], dtype=torch.int32)
    o, l = sfa_forward(q, k, v, idx, scale=0.3, dtype=torch.float64)
    for t, j in enumerate([3, 0, 2, 1]):
        for h in range(2):
            torch.testing.assert_close(o[0, t, h], v[0, j, 0], rtol=0, atol=1e-15)
            s = 0.3 * float((q[0, t, h] * k[0, j, 0]).sum())
            assert abs(float(l[0, t, h]) - s) < 1e-13


def test_closed_form_zero_query_is_mean():
    q, k, v, idx, _ = _rand_case(B=1, S=5, Hq=2, Hkv=1, K=6, seed=4)
    q.zero_()
    o, l = sfa_forward(q, k, v, idx, dtype=torch.float64)
    vm = valid_mask(idx, k.shape[1])
    for t in range(5):
        rows = idx[0, t, 0][vm[0, t, 0]].long()
        n = rows.numel()
        torch.testing.assert_close(o[0, t, 0], v[0, rows, 0].mean(0), rtol=1e-12, atol=1e-12)
        assert abs(float(l[0, t, 0]) - math.log(n)) < 1e-12


def test_duplicates_count_twice():
    """A duplicated slot is the same as one copy whose logit is raised by ln 2."""
    q, k, v, idx, _ = _rand_case(B=1, S=3, Hq=2, Hkv=1, K=4, seed=8, pad=False)
    idx[0, :, 0] = torch.tensor([[1, 2, 2, 0]] * 3, dtype=torch.int32)
    o, l = sfa_forward(q, k, v, idx, scale=0.5, dtype=torch.float64)
    for t in range(3):
        for h in range(2):
            s = torch.stack([0.5 * (q[0, t, h] * k[0, j, 0]).sum() for j in (1, 2, 0)])
            s[1] += math.log(2.0)
            w = torch.softmax(s, 0)
            ref = w[0] * v[0, 1, 0] + w[1] * v[0, 2, 0] + w[2] * v[0, 0, 0]
            torch.testing.assert_close(o[0, t, h], ref, rtol=1e-12, atol=1e-12)
            assert abs(float(l[0, t, h]) - float(torch.logsumexp(s, 0))) < 1e-12


def test_index_invariants_exact():
    """Slot permutation, padding position and the kind of invalid value do not
    change the result; unreferenced rows get exactly zero dK/dV."""
    q, k, v, idx, do = _rand_case(B=1, S=8, Skv=12, Hq=4, Hkv=2, K=6, seed=9)
    kv_lens = torch.tensor([10], dtype=torch.int32)
    o0, l0 = sfa_forward(q, k, v, idx, kv_lens=kv_lens, dtype=torch.float64)
    vm = valid_mask(idx, 12, kv_lens)
    # every invalid entry replaced by another invalid value
    for bad in (-1, -7, 10, 11, 12, 1 << 30):
        idx2 = torch.where(vm, idx, torch.full_like(idx, bad))
        o2, l2 = sfa_forward(q, k, v, idx2, kv_lens=kv_lens, dtype=torch.float64)
        assert torch.equal(o0, o2) and torch.equal(l0, l2)
    # slot permutation (fp64 sums reorder: tolerance at rounding level)
    perm = torch.randperm(6, generator=torch.Generator().manual_seed(0))
    o3, l3 = sfa_forward(q, k, v, idx[..., perm], kv_lens=kv_lens, dtype=torch.float64)
    torch.testing.assert_close(o3, o0, rtol=1e-13, atol=1e-13)
    torch.testing.assert_close(l3, l0, rtol=1e-13, atol=1e-13)
    # unreferenced key rows: zero gradient
    dq, dk, dv, _ = sfa_backward(q, k, v, idx, o0, l0, do, kv_lens=kv_lens, dtype=torch.float64)
    ref = torch.zeros(12, 2, dtype=torch.bool)
    for g in range(2):
        r = idx[0, :, g][vm[0, :, g]].long()
        ref[r, g] = True
    assert torch.all(dk[0][~ref] == 0) and torch.all(dv[0][~ref] == 0)
    assert torch.all(dk[0][ref].abs().sum(-1) > 0)


def test_fully_masked_row():
    q, k, v, idx, do = _rand_case(B=1, S=3, Hq=2, Hkv=1, K=3, seed=1)
    idx[0, 1] = -1
    o, l = sfa_forward(q, k, v, idx, dtype=torch.float64)
    assert torch.all(o[0, 1] == 0) and torch.all(torch.isneginf(l[0, 1]))
    dq, dk, dv, _ = sfa_backward(q, k, v, idx, o, l, do, dtype=torch.float64)
    assert torch.all(dq[0, 1] == 0)
    assert torch.isfinite(dk).all() and torch.isfinite(dv).all()


def test_sink_closed_form():
    q, k, v, idx, do = _rand_case(B=1, S=5, Hq=4, Hkv=2, seed=12)
    sink = torch.tensor([0.5, -2.0, 3.0, 1.0], dtype=torch.float64)
    o, l = sfa_forward(q, k, v, idx, dtype=torch.float64)
    os_, ls = sfa_forward(q, k, v, idx, sink=sink, dtype=torch.float64)
    l_ref = torch.logaddexp(l, sink.view(1, 1, 4))
    torch.testing.assert_close(ls, l_ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(os_, o * torch.exp(l - l_ref)[..., None], rtol=1e-12, atol=1e-12)
    # dsink = -Σ exp(sink - lse')·δ with δ = Σ O'·dO   (SFA.py:964-970)
    _, _, _, ds = sfa_backward(q, k, v, idx, os_, ls, do, sink=sink, dtype=torch.float64)
    delta = (os_ * do).sum(-1)
    ref = -(torch.exp(sink.view(1, 1, 4) - ls) * delta).sum((0, 1))
    torch.testing.assert_close(ds, ref, rtol=1e-12, atol=1e-12)


def test_chunking_is_invisible():
    q, k, v, idx, do = _rand_case(B=2, S=9, Hq=4, Hkv=2, seed=13)
    o1, l1 = sfa_forward(q, k, v, idx, dtype=torch.float64)
    o2, l2 = sfa_forward(q, k, v, idx, dtype=torch.float64, max_chunk_bytes=1)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    g1 = sfa_backward(q, k, v, idx, o1, l1, do, dtype=torch.float64)
    g2 = sfa_backward(q, k, v, idx, o1, l1, do, dtype=torch.float64, max_chunk_bytes=1)
    for a, b in zip(g1[:3], g2[:3]):
        torch.testing.assert_close(a, b, rtol=1e-13, atol=1e-13)


def test_planted_mistakes_are_caught():
    """Each plausible slip (wrong scale, transposed gather, natural vs base-2
    LSE, dropped mask) moves the result outside the brute-force tolerance."""
    q, k, v, idx, _ = _rand_case(seed=21)
    ob, lb = _brute_forward(q, k, v, idx, 0.37)
    o_scale, _ = sfa_forward(q, k, v, idx, scale=0.37 * 1.01, dtype=torch.float64)
    assert (o_scale - ob).abs().max() > 1e-6
    _, l_ok = sfa_forward(q, k, v, idx, scale=0.37, dtype=torch.float64)
    assert (l_ok / math.log(2) - lb).abs().max() > 1e-3     # base-2 LSE would be caught
    idx_nomask = idx.clamp(0, k.shape[1] - 1)                  # invalid slots read as row 0 / last row
    o_nm, _ = sfa_forward(q, k, v, idx_nomask, scale=0.37, dtype=torch.float64)
    assert (o_nm - ob).abs().max() > 1e-6
    v_swapped = v.flip(2)                                       # wrong KV head for the group
    o_sw, _ = sfa_forward(q, k, v_swapped, idx, scale=0.37, dtype=torch.float64)
    assert (o_sw - ob).abs().max() > 1e-6


def test_count_valid_pairs():
    idx = torch.tensor([[[[0, -1, 5, 9]], [[2, 3, -1, -1]]]], dtype=torch.int32)
    assert count_valid_pairs(idx, 6) == 4
    assert count_valid_pairs(idx, 6, torch.tensor([3], dtype=torch.int32)) == 2


def test_autograd_restatement_forward_matches_brute_force():
    q, k, v, idx, _ = _rand_case(B=2, S=6, Skv=9, seed=31)
    kv_lens = torch.tensor([7, 9], dtype=torch.int32)
    sink = torch.tensor([0.2, -0.4, 1.1, 0.0], dtype=torch.float64)
    for s_ in (None, sink):
        o, l = sfa_forward_autograd(q, k, v, idx, scale=0.45, kv_lens=kv_lens, sink=s_)
        ob, lb = _brute_forward(q, k, v, idx, 0.45, kv_lens=kv_lens, sink=s_)
        torch.testing.assert_close(o, ob, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(l, lb, rtol=1e-12, atol=1e-12)
