"""GPU parity of the top-k index producer (``sfa_indexer_topk``).

* Scores: against the oracle's fp32 evaluation of the same bf16 inputs
  (relative max error <= 1e-4 of the row's largest magnitude).
* Selection: exact.  Given the kernel's own scores, the oracle's selection
  (score descending, equal scores by key, then ascending key order) must give
  bitwise the same index rows, including rows with exact ties and rows with
  fewer visible keys than k.
* End to end: against the oracle's scores every selected key is visible and
  distinct, and no unselected visible key beats a selected one by more than
  the score tolerance.
* Consumer: the produced rows drive the MLA forward, checked against the
  sparse attention oracle."""
import math
import sys

import pytest
import torch

import ops_amd
from oracle.sfa_oracle import indexer_key_end, indexer_scores, indexer_topk
from oracle.sfa_oracle import sfa_forward as ref_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCORE_RTOL = 1e-4


def _say(msg):
    print(f"\n[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _inputs(B, Sq, Skv, H, seed, dup_keys=False):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    q = torch.randn(B, Sq, H, 128, generator=g, device=DEV).bfloat16()
    k = torch.randn(B, Skv, 128, generator=g, device=DEV).bfloat16()
    if dup_keys:  # every key repeated 4 times: exact score ties
        k = k[:, ::4].repeat_interleave(4, dim=1)[:, :Skv].contiguous()
    w = torch.randn(B, Sq, H, generator=g, device=DEV) / math.sqrt(H)
    return q, k, w


def _check_rows(idx, scores_ref, end, K, tol):
    """Structure + near-optimality against the oracle's scores."""
    B, Sq = end.shape
    for b in range(B):
        for t in range(Sq):
            n = int(end[b, t])
            row = idx[b, t, 0]
            m = min(n, K)
            sel = row[:m]
            assert bool((row[m:] == -1).all()), (b, t)
            assert bool((sel >= 0).all()) and bool((sel < n).all()), (b, t)
            assert bool((sel[1:] > sel[:-1]).all()), (b, t)  # ascending, distinct
            if n > K:
                sc = scores_ref[b, t, :n]
                mask = torch.ones(n, dtype=torch.bool)
                mask[sel.long()] = False
                assert float(sc[mask].max()) <= float(sc[sel.long()].min()) + tol, (b, t)


@pytest.mark.parametrize("H,K,kv,dup", [
    (64, 16, None, False),
    (64, 64, [300, 180], False),
    (32, 40, [250, 300], False),
    (128, 16, None, False),
    (64, 32, None, True),
], ids=["h64-k16", "h64-k64-kvlens", "h32-k40-kvlens", "h128-k16", "h64-ties"])
def test_indexer_small(H, K, kv, dup):
    B, Sq, Skv = 2, 100, 300
    _say(f"indexer B={B} Sq={Sq} Skv={Skv} H={H} K={K} kv_lens={kv} ties={dup}")
    q, k, w = _inputs(B, Sq, Skv, H, seed=H + K, dup_keys=dup)
    kv_lens = torch.tensor(kv, dtype=torch.int32, device=DEV) if kv else None
    idx, logits = ops_amd.indexer_topk(q, k, w, K, kv_lens=kv_lens, return_logits=True)
    torch.cuda.synchronize()
    idx, logits = idx.cpu(), logits.cpu()
    end = indexer_key_end(B, Sq, Skv, None if kv_lens is None else kv_lens.cpu())
    ref = indexer_scores(q.cpu(), k.cpu(), w.cpu(), None if kv_lens is None else kv_lens.cpu())
    vis = torch.arange(Skv)[None, None, :] < end[:, :, None]
    scale = float(ref[vis].abs().max())
    err = float((logits[vis] - ref[vis]).abs().max())
    assert err <= SCORE_RTOL * scale, f"score error {err} vs scale {scale}"
    # exact selection from the kernel's own scores
    own = torch.where(vis, logits, torch.full_like(logits, -math.inf))
    assert torch.equal(idx, indexer_topk(own, K, end))
    _check_rows(idx, ref, end, K, 2 * SCORE_RTOL * scale)


def test_indexer_prefill_full_size_rows():
    # the DeepSeek-V3.2 prefill shape: S = 32768, 64 index heads, top-k 2048
    B, S, H, K = 1, 32768, 64, 2048
    _say(f"indexer full prefill S={S} H={H} K={K}")
    q, k, w = _inputs(B, S, S, H, seed=5)
    idx, logits = ops_amd.indexer_topk(q, k, w, K, return_logits=True)
    torch.cuda.synchronize()
    end = indexer_key_end(B, S, S)
    rows = [0, 1, 2046, 2047, 2048, 2049, 5000, 17011, 32767]
    own = logits[0, rows].cpu()
    vis = torch.arange(S)[None, :] < end[0, rows][:, None]
    own = torch.where(vis, own, torch.full_like(own, -math.inf))
    got = idx[0, rows].cpu()
    assert torch.equal(got[:, None], indexer_topk(own[None], K, end[:, rows])[0][:, None])
    # scores of the last three sampled rows against a direct fp32 evaluation
    for i, r in enumerate(rows[-3:], len(rows) - 3):
        ref = _ref_row(q, k, w, 0, r, r + 1)
        assert float((own[i, :r + 1] - ref).abs().max()) <= SCORE_RTOL * float(ref.abs().max())
    # every row: ascending, in range, padded exactly where the prefix is short
    full = idx[0, :, 0]
    n = torch.clamp(torch.arange(S, device=DEV) + 1, max=K)
    valid = full >= 0
    assert torch.equal(valid.sum(-1), n)
    assert bool(((full[:, 1:] > full[:, :-1]) | ~valid[:, 1:]).all())
    assert bool((full < (torch.arange(S, device=DEV) + 1)[:, None]).all())


def _ref_row(q, k, w, b, t, end):
    """fp32 scores of query t of sequence b over keys [0, end)."""
    qr = q[b, t].cpu().float()
    kr = k[b, :end].cpu().float()
    return (w[b, t].cpu()[:, None] * (qr @ kr.T).clamp_min(0)).sum(0)


def test_indexer_decode_shape():
    # one query per sequence over contexts of 16K-64K keys (the decode shape)
    B, Skv, H, K = 64, 65536, 64, 2048
    _say(f"indexer decode B={B} Skv={Skv} H={H} K={K}")
    q, k, w = _inputs(B, 1, Skv, H, seed=9)
    g = torch.Generator(device=DEV)
    g.manual_seed(3)
    kv_lens = torch.randint(1000, Skv + 1, (B,), generator=g, device=DEV, dtype=torch.int32)
    kv_lens[0] = 100  # fewer keys than k
    idx, logits = ops_amd.indexer_topk(q, k, w, K, kv_lens=kv_lens, return_logits=True)
    torch.cuda.synchronize()
    end = indexer_key_end(B, 1, Skv, kv_lens.cpu())
    own = logits.cpu()
    vis = torch.arange(Skv)[None, None, :] < end[:, :, None]
    own = torch.where(vis, own, torch.full_like(own, -math.inf))
    assert torch.equal(idx.cpu(), indexer_topk(own, K, end))
    for b in (1, 7, 63):
        ref = _ref_row(q, k, w, b, 0, int(end[b, 0]))
        sc = own[b, 0, :int(end[b, 0])]
        assert float((sc - ref).abs().max()) <= SCORE_RTOL * float(ref.abs().max())


@pytest.mark.parametrize("H,fp8,Sq", [(64, False, 5), (32, False, 5), (128, False, 5), (64, True, 5),
                                      (64, False, 1), (64, False, 2), (32, False, 1), (64, True, 1), (32, True, 2),
                                      (128, False, 1)],
                         ids=["h64", "h32", "h128", "h64-fp8", "1q-h64", "1q-h64-sq2", "1q-h32", "1q-h64-fp8",
                              "1q-h32-fp8-sq2", "1q-h128"])
def test_indexer_key_splits(H, fp8, Sq):
    """Launches with few queries split each query's (or query block's) keys
    over several workgroups: 3 sequences of up to 5000 keys, kv_lens that end
    one sequence inside its third split of 1024 keys and leave another only
    part of its first tile (the later splits exit at once).  With 5 queries
    per sequence the block kernel runs (5 splits per block); with 1 or 2 the
    one-query kernel (splits of 8 tiles, each wave streaming its own tiles,
    a wave with no tile idle).  Every visible score against the oracle, the
    selection exact."""
    B, Skv, K = 3, 5000, 100
    _say(f"indexer key splits B={B} Sq={Sq} Skv={Skv} H={H} K={K} fp8={fp8}")
    kv_lens = torch.tensor([5000, 2100, 40], dtype=torch.int32, device=DEV)
    ks = None
    if fp8:
        q, k, w, ks = _fp8_inputs(B, Sq, Skv, H, seed=31)
    else:
        q, k, w = _inputs(B, Sq, Skv, H, seed=31 + H)
    idx, logits = ops_amd.indexer_topk(q, k, w, K, kv_lens=kv_lens, return_logits=True, k_scale=ks)
    torch.cuda.synchronize()
    idx, logits = idx.cpu(), logits.cpu()
    end = indexer_key_end(B, Sq, Skv, kv_lens.cpu())
    ref = indexer_scores(q.cpu().float(), k.cpu().float(), w.cpu(), kv_lens.cpu(),
                         k_scale=None if ks is None else ks.cpu())
    vis = torch.arange(Skv)[None, None, :] < end[:, :, None]
    scale = float(ref[vis].abs().max())
    err = float((logits[vis] - ref[vis]).abs().max())
    assert err <= SCORE_RTOL * scale, f"score error {err} vs scale {scale}"
    own = torch.where(vis, logits, torch.full_like(logits, -math.inf))
    assert torch.equal(idx, indexer_topk(own, K, end))
    _check_rows(idx, ref, end, K, 2 * SCORE_RTOL * scale)


@pytest.mark.parametrize("pattern", ["sawtooth", "sorted", "clustered"])
def test_indexer_selection_position_patterns(pattern):
    """Rows of 5000 scores whose values follow the key position (the
    selection kernel holds them as runs of 8 per thread): a sawtooth of
    period 8 (every run holds one score of each of 8 levels), an ascending
    row, and runs of 8 in 8 tight clusters (many near ties around the
    threshold, decided by the low bits).  The selection is exact against the
    oracle's on the kernel's own scores, and the scores match the oracle."""
    B, Sq, Skv, H, K = 2, 1, 5000, 64, 100
    _say(f"indexer selection position patterns: {pattern}")
    g = torch.Generator(device="cpu")
    g.manual_seed(17)
    d = torch.randn(128, generator=g)
    d = d / d.norm()
    pos = torch.arange(Skv, dtype=torch.float32)
    if pattern == "sawtooth":
        amp = (pos % 8) + 1.0
    elif pattern == "sorted":
        amp = 1.0 + pos / Skv
    else:
        amp = 1.0 + ((pos // 8) % 8) * 0.25
    noise = 1e-2 * torch.randn(B, Skv, 128, generator=g)
    k = (amp[None, :, None] * d[None, None, :] + noise).bfloat16()
    q = (d[None, None, None, :].expand(B, Sq, H, 128) + 0.1 * torch.randn(B, Sq, H, 128, generator=g)).bfloat16()
    w = torch.rand(B, Sq, H, generator=g) / H
    q, k, w = q.to(DEV), k.to(DEV), w.to(DEV)
    idx, logits = ops_amd.indexer_topk(q, k, w, K, return_logits=True)
    torch.cuda.synchronize()
    idx, logits = idx.cpu(), logits.cpu()
    end = indexer_key_end(B, Sq, Skv)
    ref = indexer_scores(q.cpu(), k.cpu(), w.cpu())
    scale = float(ref.abs().max())
    assert float((logits - ref).abs().max()) <= SCORE_RTOL * scale
    assert torch.equal(idx, indexer_topk(logits, K, end))
    _check_rows(idx, ref, end, K, 2 * SCORE_RTOL * scale)


@pytest.mark.parametrize("K,kv,dup", [(301, [20000, 250], False), (300, [17000, 9000], True),
                                       (2048, [20000, 12000], False)],
                         ids=["k301-short-row", "k300-ties", "k2048"])
def test_indexer_segmented_selection(K, kv, dup):
    """Launches of few long rows (under 256 rows of at least 16384 keys) select
    in two phases: each row cut into segments whose own top-k become the
    row's candidate lists (padded to a multiple of 4 with -1), then the top-k
    of the candidates.  Here 2 sequences x 3 queries of up to 20000 keys:
    8 segments of 2528 keys, a row shorter than k (no segment selects), a
    row ending in its fourth segment (empty segments), exact ties (keys
    repeated 4 times), and k = 2048 (segments shorter than k: all their keys
    are candidates).  Every visible score against the oracle, the selection
    exact against the oracle's on the kernel's own scores."""
    B, Sq, Skv, H = 2, 3, 20000, 64
    _say(f"indexer segmented selection B={B} Sq={Sq} Skv={Skv} K={K} kv_lens={kv} ties={dup}")
    q, k, w = _inputs(B, Sq, Skv, H, seed=K, dup_keys=dup)
    kv_lens = torch.tensor(kv, dtype=torch.int32, device=DEV)
    idx, logits = ops_amd.indexer_topk(q, k, w, K, kv_lens=kv_lens, return_logits=True)
    torch.cuda.synchronize()
    idx, logits = idx.cpu(), logits.cpu()
    end = indexer_key_end(B, Sq, Skv, kv_lens.cpu())
    ref = indexer_scores(q.cpu(), k.cpu(), w.cpu(), kv_lens.cpu())
    vis = torch.arange(Skv)[None, None, :] < end[:, :, None]
    scale = float(ref[vis].abs().max())
    err = float((logits[vis] - ref[vis]).abs().max())
    assert err <= SCORE_RTOL * scale, f"score error {err} vs scale {scale}"
    own = torch.where(vis, logits, torch.full_like(logits, -math.inf))
    assert torch.equal(idx, indexer_topk(own, K, end))
    _check_rows(idx, ref, end, K, 2 * SCORE_RTOL * scale)


def test_indexer_feeds_mla_forward():
    # producer -> consumer: index rows from the indexer drive the MLA forward
    B, S, Hq, K, H = 1, 384, 128, 64, 64
    _say(f"indexer -> MLA forward S={S} K={K}")
    q_i, k_i, w_i = _inputs(B, S, S, H, seed=21)
    idx = ops_amd.indexer_topk(q_i, k_i, w_i, K)
    g = torch.Generator(device=DEV)
    g.manual_seed(22)
    q = torch.randn(B, S, Hq, 576, generator=g, device=DEV).bfloat16()
    kv = torch.randn(B, S, 1, 576, generator=g, device=DEV).bfloat16()
    scale = 1.0 / math.sqrt(576)
    out, lse = ops_amd.sfa_forward(q, kv, kv[..., :512], idx, scale)
    torch.cuda.synchronize()
    o_ref, l_ref = ref_forward(q.cpu().float(), kv.cpu().float(), kv[..., :512].cpu().float(), idx.cpu(), scale)
    assert float((out.float().cpu() - o_ref).abs().max()) <= 2e-2
    assert float((lse.cpu() - l_ref).abs().max()) <= 1e-3


def test_indexer_degenerate_rows():
    # more queries than keys (early rows see nothing), a zero-length sequence,
    # top-k larger than the whole context
    B, Sq, Skv, H, K = 3, 64, 40, 64, 50
    _say(f"indexer degenerate rows B={B} Sq={Sq} Skv={Skv} K={K}")
    q, k, w = _inputs(B, Sq, Skv, H, seed=31)
    kv_lens = torch.tensor([0, 40, 17], dtype=torch.int32, device=DEV)
    idx = ops_amd.indexer_topk(q, k, w, K, kv_lens=kv_lens).cpu()
    torch.cuda.synchronize()
    end = indexer_key_end(B, Sq, Skv, kv_lens.cpu())
    assert int(end[0].max()) == 0 and int(end[1, 0]) == 0 and int(end[1, -1]) == 40
    ref = indexer_topk(indexer_scores(q.cpu(), k.cpu(), w.cpu(), kv_lens.cpu()), K, end)
    assert torch.equal(idx, ref)  # every row keeps all of its (<= K) visible keys
    assert bool((idx[0] == -1).all())


def _fp8_inputs(B, Sq, Skv, H, seed):
    """fp8 e4m3 q / k as DeepSeek-V3.2 stores them: per-token k scales, the
    per-(token, head) q scales folded into the weights."""
    q, k, w = _inputs(B, Sq, Skv, H, seed)
    f8 = torch.float8_e4m3fn
    ks = k.float().abs().amax(-1).clamp_min(1e-6) / 448.0
    k8 = (k.float() / ks[..., None]).to(f8)
    qs = q.float().abs().amax(-1).clamp_min(1e-6) / 448.0
    q8 = (q.float() / qs[..., None]).to(f8)
    return q8, k8, (w * qs).contiguous(), ks.contiguous()


@pytest.mark.parametrize("H,K,kv", [(64, 32, None), (64, 48, [300, 170]), (32, 16, None), (128, 40, [250, 300])],
                         ids=["h64", "h64-kvlens", "h32", "h128-kvlens"])
def test_indexer_fp8_small(H, K, kv):
    B, Sq, Skv = 2, 100, 300
    _say(f"indexer fp8 B={B} Sq={Sq} Skv={Skv} H={H} K={K} kv_lens={kv}")
    q8, k8, w, ks = _fp8_inputs(B, Sq, Skv, H, seed=7 * H + K)
    kv_lens = torch.tensor(kv, dtype=torch.int32, device=DEV) if kv else None
    idx, logits = ops_amd.indexer_topk(q8, k8, w, K, kv_lens=kv_lens, return_logits=True, k_scale=ks)
    torch.cuda.synchronize()
    idx, logits = idx.cpu(), logits.cpu()
    kvc = None if kv_lens is None else kv_lens.cpu()
    end = indexer_key_end(B, Sq, Skv, kvc)
    ref = indexer_scores(q8.cpu().float(), k8.cpu().float(), w.cpu(), kvc, k_scale=ks.cpu())
    vis = torch.arange(Skv)[None, None, :] < end[:, :, None]
    scale = float(ref[vis].abs().max())
    err = float((logits[vis] - ref[vis]).abs().max())
    assert err <= SCORE_RTOL * scale, f"score error {err} vs scale {scale}"
    own = torch.where(vis, logits, torch.full_like(logits, -math.inf))
    assert torch.equal(idx, indexer_topk(own, K, end))
    _check_rows(idx, ref, end, K, 2 * SCORE_RTOL * scale)


def test_indexer_fp8_prefill_full_size_rows():
    B, S, H, K = 1, 32768, 64, 2048
    _say(f"indexer fp8 full prefill S={S} H={H} K={K}")
    q8, k8, w, ks = _fp8_inputs(B, S, S, H, seed=15)
    idx, logits = ops_amd.indexer_topk(q8, k8, w, K, return_logits=True, k_scale=ks)
    torch.cuda.synchronize()
    end = indexer_key_end(B, S, S)
    rows = [0, 2047, 2048, 9000, 32767]
    own = logits[0, rows].cpu()
    vis = torch.arange(S)[None, :] < end[0, rows][:, None]
    own = torch.where(vis, own, torch.full_like(own, -math.inf))
    assert torch.equal(idx[0, rows].cpu()[:, None], indexer_topk(own[None], K, end[:, rows])[0][:, None])
    r = 32767
    qr, kr = q8[0, r].cpu().float(), k8[0].cpu().float()
    ref = (w[0, r].cpu()[:, None] * (qr @ kr.T).clamp_min(0)).sum(0) * ks[0].cpu()
    assert float((own[-1] - ref).abs().max()) <= SCORE_RTOL * float(ref.abs().max())
