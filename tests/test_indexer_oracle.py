"""The top-k index producer's oracle (``indexer_scores``, ``indexer_topk``)
pinned without restating it: a pure-Python fp64 loop for the scores, a
brute-force enumeration of each row's best keys with the tie rule spelled out
(score descending, then key ascending), closed forms (one-hot keys, a single
head), exact ties, the visibility rule for prefill / decode / short
sequences, and planted mistakes (no ReLU, the opposite tie rule) that the
loops must catch.  Host and C-ABI checks of ``indexer_topk`` need no GPU."""
import ctypes
import math
import random

import pytest
import torch

import ops_amd
from ops_amd import _lib
from oracle.sfa_oracle import indexer_key_end, indexer_scores, indexer_topk


def _loop_scores(q, k, w, end):
    B, Sq, H, D = q.shape
    Skv = k.shape[1]
    out = torch.full((B, Sq, Skv), -math.inf, dtype=torch.float64)
    for b in range(B):
        for t in range(Sq):
            for s in range(int(end[b, t])):
                tot = 0.0
                for h in range(H):
                    dot = sum(float(q[b, t, h, d]) * float(k[b, s, d]) for d in range(D))
                    tot += float(w[b, t, h]) * max(dot, 0.0)
                out[b, t, s] = tot
    return out


def _loop_topk(scores, K, end):
    B, Sq, _ = scores.shape
    out = torch.full((B, Sq, 1, K), -1, dtype=torch.int32)
    for b in range(B):
        for t in range(Sq):
            n = int(end[b, t])
            keys = sorted(range(n), key=lambda s: (-float(scores[b, t, s]), s))[:K]
            for j, s in enumerate(sorted(keys)):
                out[b, t, 0, j] = s
    return out


def _case(seed, B=2, Sq=5, Skv=9, H=3, D=4):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, H, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Skv, D, generator=g, dtype=torch.float64)
    w = torch.randn(B, Sq, H, generator=g, dtype=torch.float64)
    return q, k, w


def test_key_end_rule():
    assert indexer_key_end(1, 4, 4).tolist() == [[1, 2, 3, 4]]                   # causal prefill
    assert indexer_key_end(2, 1, 10, torch.tensor([7, 12])).tolist() == [[7], [10]]  # decode: the context
    assert indexer_key_end(1, 3, 8).tolist() == [[6, 7, 8]]                      # chunk at the end of a prefix
    assert indexer_key_end(1, 4, 8, torch.tensor([2])).tolist() == [[0, 0, 1, 2]]  # shorter than the queries


@pytest.mark.parametrize("seed", range(3))
def test_scores_match_loop(seed):
    q, k, w = _case(seed)
    kv = torch.tensor([9, 6])
    end = indexer_key_end(2, 5, 9, kv)
    got = indexer_scores(q, k, w, kv, dtype=torch.float64)
    ref = _loop_scores(q, k, w, end)
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), fin)
    assert torch.allclose(got[fin], ref[fin], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("K", [1, 3, 6, 20])
def test_topk_matches_enumeration_with_ties(K):
    rng = random.Random(K)
    B, Sq, Skv = 2, 6, 12
    scores = torch.tensor([[[float(rng.randrange(4)) for _ in range(Skv)] for _ in range(Sq)] for _ in range(B)],
                          dtype=torch.float64)  # few distinct values: many exact ties
    end = torch.tensor([[rng.randrange(0, Skv + 1) for _ in range(Sq)] for _ in range(B)])
    assert torch.equal(indexer_topk(scores, K, end), _loop_topk(scores, K, end))


def test_closed_form_one_hot_keys():
    # k_s = e_s, one head with weight 1: the score of key s is relu(q[s])
    D = 8
    q = torch.tensor([3.0, -1.0, 5.0, 0.5, 4.0, -2.0, 2.0, 1.0], dtype=torch.float64).view(1, 1, 1, D)
    k = torch.eye(D, dtype=torch.float64).view(1, D, D)
    w = torch.ones(1, 1, 1, dtype=torch.float64)
    sc = indexer_scores(q, k, w, dtype=torch.float64)
    assert sc.view(-1).tolist() == [3.0, 0.0, 5.0, 0.5, 4.0, 0.0, 2.0, 1.0]
    idx = indexer_topk(sc, 3, indexer_key_end(1, 1, D))
    assert idx.view(-1).tolist() == [0, 2, 4]


def test_planted_mistakes_are_caught():
    q, k, w = _case(7)
    end = indexer_key_end(2, 5, 9)
    ref = _loop_scores(q, k, w, end)
    fin = torch.isfinite(ref)
    no_relu = torch.einsum("bth,bths->bts", w, torch.einsum("bthd,bsd->bths", q, k))
    assert not torch.allclose(no_relu[fin], ref[fin])
    # the opposite tie rule (higher key first) picks different keys on ties
    scores = torch.zeros(1, 1, 6, dtype=torch.float64)
    e = torch.tensor([[6]])
    assert indexer_topk(scores, 2, e).view(-1).tolist() == [0, 1]
    assert _loop_topk(scores, 2, e).view(-1).tolist() == [0, 1]


def test_host_validation():
    q = torch.randn(1, 4, 64, 128).bfloat16()
    k = torch.randn(1, 8, 128).bfloat16()
    w = torch.randn(1, 4, 64)
    with pytest.raises(ValueError, match="GPU"):
        ops_amd.indexer_topk(q, k, w, 4)
    with pytest.raises(ValueError):
        ops_amd.indexer_topk(q, k[:, :, :64], w, 4)
    with pytest.raises(ValueError):
        ops_amd.indexer_topk(q, k, w, 0)


def _valid_indexer_args():
    a = _lib.IndexerArgs()
    a.B, a.Sq, a.Skv, a.H, a.D, a.topk = 1, 4, 8, 64, 128, 4
    a.dtype = _lib.SFA_DTYPE_BF16
    for name in ("q", "k", "w", "idx"):
        setattr(a, name, 0x10000)
    a.q_sh, a.q_ss, a.q_sb = 128, 64 * 128, 4 * 64 * 128
    a.k_ss, a.k_sb = 128, 8 * 128
    return a


@pytest.mark.parametrize("field,value,code", [
    ("topk", 0, _lib.SFA_E_INVALID), ("B", 0, _lib.SFA_E_INVALID), ("q", None, _lib.SFA_E_INVALID),
    ("flags", 1, _lib.SFA_E_INVALID), ("D", 64, _lib.SFA_E_UNSUPPORTED), ("H", 48, _lib.SFA_E_UNSUPPORTED),
    ("Skv", 65537, _lib.SFA_E_UNSUPPORTED), ("k_ss", 100, _lib.SFA_E_INVALID), ("q", 0x10008, _lib.SFA_E_INVALID),
    ("dtype", 0, _lib.SFA_E_INVALID), ("k_scale", 0x10000, _lib.SFA_E_INVALID),
])
def test_indexer_abi_rejects(field, value, code):
    lib = _lib.load()
    a = _valid_indexer_args()
    setattr(a, field, value)
    assert lib.sfa_indexer_topk(ctypes.byref(a), None, 0, None) == code
    assert lib.sfa_last_error()
    assert lib.sfa_indexer_topk_workspace_size(ctypes.byref(a)) == 0


def test_indexer_workspace_is_bounded():
    lib = _lib.load()
    a = _valid_indexer_args()
    a.Sq, a.Skv = 32768, 32768
    a.q_ss, a.q_sb = 64 * 128, 32768 * 64 * 128
    a.k_sb = 32768 * 128
    ws = lib.sfa_indexer_topk_workspace_size(ctypes.byref(a))
    assert 0 < ws <= (1 << 30) + 4096
    a.logits = 0x10000
    a.g_ss, a.g_sb = 32768, 32768 * 32768
    assert lib.sfa_indexer_topk_workspace_size(ctypes.byref(a)) == 0
    assert lib.sfa_indexer_topk(None, None, 0, None) == _lib.SFA_E_INVALID


def test_indexer_workspace_decode_step():
    # 64 sequences x 1 query over 65536 keys: one score row per sequence, and
    # the candidate lists of the two-phase selection (4 segments per row,
    # ids + order keys), also when the caller holds the scores
    lib = _lib.load()
    a = _valid_indexer_args()
    a.B, a.Sq, a.Skv, a.topk = 64, 1, 65536, 2048
    a.q_sb, a.q_ss = 64 * 128, 64 * 128
    a.k_sb = 65536 * 128
    a.w_sb, a.w_ss = 64, 64
    a.i_sb, a.i_ss = 2048, 2048
    cand = 2 * 64 * 4 * 2048 * 4
    assert lib.sfa_indexer_topk_workspace_size(ctypes.byref(a)) == 64 * 65536 * 4 + cand
    a.logits = 0x10000
    a.g_ss, a.g_sb = 65536, 65536
    assert lib.sfa_indexer_topk_workspace_size(ctypes.byref(a)) == cand
    # a long prefill row set takes no candidates
    a.B, a.Sq = 1, 4096
    a.q_sb, a.w_sb, a.i_sb, a.g_sb = 4096 * 64 * 128, 4096 * 64, 4096 * 2048, 4096 * 65536
    assert lib.sfa_indexer_topk_workspace_size(ctypes.byref(a)) == 0


def test_fp8_key_scale_closed_form():
    # a positive per-key scale multiplies that key's score (relu commutes with it)
    q, k, w = _case(3)
    ks = torch.rand(2, 9, dtype=torch.float64) + 0.5
    end = indexer_key_end(2, 5, 9)
    scaled = indexer_scores(q, k, w, dtype=torch.float64, k_scale=ks)
    plain = _loop_scores(q, k * ks[..., None], w, end)
    fin = torch.isfinite(plain)
    assert torch.allclose(scaled[fin], plain[fin], rtol=1e-12, atol=1e-12)


def test_fp8_indexer_abi_accepts_fp8_strides():
    lib = _lib.load()
    a = _valid_indexer_args()
    a.dtype = _lib.SFA_DTYPE_FP8_E4M3
    a.k_ss, a.k_sb = 144, 8 * 144          # 144 B rows: a multiple of 16 bytes in fp8
    assert lib.sfa_indexer_topk_workspace_size(ctypes.byref(a)) > 0
    a.k_ss = 132                            # not a multiple of 16 bytes
    assert lib.sfa_indexer_topk(ctypes.byref(a), None, 0, None) == _lib.SFA_E_INVALID
