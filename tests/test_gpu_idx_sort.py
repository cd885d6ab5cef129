"""GPU tests of the index-row sort that sfa_fwd runs ahead of the persistent
MLA prefill (sfa_idx_sort.hip), called through the C ABI.

The sort only reorders a row's slots: valid keys (0 <= key < bound, bound =
kv_lens[b] or Skv) ascending, then -1, and a row that repeats a key stays as
it is.  The expected rows are computed here on the host from that rule, and
the forward on the caller's rows (sort pass) must then be bitwise the forward
on the host-sorted rows with SFA_FWD_IDX_SORTED set (no pass): both run the
same kernel on the same slots, so any slot the pass dropped, repeated,
misplaced or let through out of range changes some row of the output.  The
rows include repeated keys, keys at and beyond kv_lens, padding values other
than -1, rows with no valid key, short causal rows, keys beyond the first
bitmap half (Skv > 32768) up to Skv = 65536, and a top-k of 100.  Sampled rows are also checked
against the CPU oracle (O max-abs 2e-2, LSE 1e-3)."""
import math
import sys

import pytest
import torch

import ops_amd
from oracle.sfa_oracle import sfa_forward as ref_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(f"\n[gpu] {msg}", flush=True)
    sys.stdout.flush()


def host_sorted(idx, bounds):
    """The pass's rule on the host: per row, the valid keys ascending then -1;
    rows that repeat a valid key unchanged."""
    out = idx.clone()
    B, S, H, K = idx.shape
    for b in range(B):
        x = idx[b].reshape(-1, K)
        valid = (x >= 0) & (x < int(bounds[b]))
        big = torch.iinfo(torch.int32).max
        keyed = torch.where(valid, x, torch.full_like(x, big))
        srt = torch.sort(keyed, dim=1).values
        # a repeat shows as two equal neighbours among the sorted valid keys
        rep = ((srt[:, 1:] == srt[:, :-1]) & (srt[:, 1:] != big)).any(dim=1)
        srt = torch.where(srt == big, torch.full_like(srt, -1), srt)
        x_new = torch.where(rep[:, None], x, srt)
        out[b] = x_new.reshape(S, H, K)
    return out


def _case(B, S, Skv, K, seed, Hkv=1):
    g = torch.Generator(device="cpu").manual_seed(seed)
    Hq = 128 * Hkv
    q = torch.randn(B, S, Hq, 576, generator=g).bfloat16()
    kv = torch.randn(B, Skv, Hkv, 576, generator=g).bfloat16()
    idx = torch.full((B, S, Hkv, K), -1, dtype=torch.int32)
    for b in range(B):
        for t in range(S):
            # causal prefix of a query placed at the end of the context
            top = Skv - S + t + 1
            n = min(K, top)
            for h in range(Hkv):
                idx[b, t, h, :n] = torch.randperm(top, generator=g)[:n].to(torch.int32)
    return q, kv, idx


def _plant(idx, bounds, seed):
    """Rows the rule treats specially: repeats, keys >= bound, odd padding,
    empty rows, padding in the middle of a row."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    B, S, H, K = idx.shape
    rows = torch.randperm(S, generator=g)[:40].tolist()
    for j, t in enumerate(rows):
        b = j % B
        r = idx[b, t, j % H]
        kind = j % 5
        if kind == 0:    # a repeated key (row stays in its own order)
            r[5] = r[1]
        elif kind == 1:  # keys at and beyond the bound, and far beyond Skv
            r[0] = int(bounds[b])
            r[3] = int(bounds[b]) + 7
            r[9] = 1 << 30
        elif kind == 2:  # padding other than -1, inside the row
            r[2] = -7
            r[K // 2] = -(1 << 31)
        elif kind == 3:  # no valid key at all
            r[:] = -1
            r[K - 1] = -3
        else:            # a repeat of an invalid key is no repeat
            r[4] = -1
            r[6] = -1
    return idx


@pytest.mark.parametrize("B,S,Skv,K,lens", [
    (2, 2080, 2080, 256, (2080, 1500)),   # 4160 items: persistent, kv_lens, causal short rows
    (1, 4100, 40000, 512, None),          # Skv > 32768: the 2048-word bitmap
    (1, 4096, 65536, 100, None),          # the bitmap's last word, top-k not a multiple of the slots per thread
])
def test_sorted_pass_is_bitwise_the_host_sorted_forward(B, S, Skv, K, lens):
    _say(f"index sort: B={B} S={S} Skv={Skv} K={K} kv_lens={lens}")
    q, kv, idx = _case(B, S, Skv, K, seed=11 + S)
    bounds = torch.tensor(lens if lens else (Skv,) * B, dtype=torch.int32)
    idx = _plant(idx, bounds, seed=5)
    exp = host_sorted(idx, bounds)
    assert not torch.equal(exp, idx)
    scale = 1.0 / math.sqrt(576)
    dq, dkv, di, de = (t.to(DEV) for t in (q, kv, idx, exp))
    dl = bounds.to(DEV) if lens else None
    o_a, l_a = ops_amd.sfa_forward(dq, dkv, dkv[..., :512], di, scale, kv_lens=dl)
    o_b, l_b = ops_amd.sfa_forward(dq, dkv, dkv[..., :512], de, scale, kv_lens=dl, idx_sorted=True)
    torch.cuda.synchronize()
    assert torch.equal(o_a, o_b) and torch.equal(l_a, l_b)
    # the caller's rows were not written
    assert torch.equal(di.cpu(), idx)
    rows = torch.tensor([0, 1, 17, S // 2, S - 2, S - 1])
    kl = bounds if lens else None
    o_ref, l_ref = ref_forward(q[:, rows].float(), kv.float(), kv[..., :512].float(), idx[:, rows], scale,
                               kv_lens=kl)
    err_o = float((o_a[:, rows].float().cpu() - o_ref).abs().max())
    finite = torch.isfinite(l_ref)
    assert torch.equal(torch.isfinite(l_a[:, rows].cpu()), finite)
    err_l = float((l_a[:, rows].cpu()[finite] - l_ref[finite]).abs().max())
    assert err_o <= 2e-2 and err_l <= 1e-3, (err_o, err_l)


def test_sorted_pass_two_kv_heads_strided_rows():
    """Two KV heads (Hq = 256, 128 heads each) and index rows read through a
    strided view (head stride K + 48, a padded last dimension): the pass
    decodes (b, t, g) from its row number and reads the caller's strides;
    bitwise the forward on host-sorted rows, sampled rows against the
    oracle."""
    B, S, Skv, K, H = 1, 2080, 3000, 256, 2
    _say(f"index sort: B={B} S={S} Skv={Skv} K={K} Hkv={H}, strided index rows")
    q, kv, idx = _case(B, S, Skv, K, seed=29, Hkv=H)
    bounds = torch.tensor([Skv], dtype=torch.int32)
    idx = _plant(idx, bounds, seed=9)
    exp = host_sorted(idx, bounds)
    wide = torch.full((B, S, H, K + 48), 7, dtype=torch.int32)
    wide[..., :K] = idx
    scale = 1.0 / math.sqrt(576)
    dq, dkv, de = (t.to(DEV) for t in (q, kv, exp))
    di = wide.to(DEV)[..., :K]
    assert di.stride() == (S * H * (K + 48), H * (K + 48), K + 48, 1)
    o_a, l_a = ops_amd.sfa_forward(dq, dkv, dkv[..., :512], di, scale)
    o_b, l_b = ops_amd.sfa_forward(dq, dkv, dkv[..., :512], de, scale, idx_sorted=True)
    torch.cuda.synchronize()
    assert torch.equal(o_a, o_b) and torch.equal(l_a, l_b)
    rows = torch.tensor([0, 5, S // 3, S - 1])
    o_ref, l_ref = ref_forward(q[:, rows].float(), kv.float(), kv[..., :512].float(), idx[:, rows], scale)
    err_o = float((o_a[:, rows].float().cpu() - o_ref).abs().max())
    finite = torch.isfinite(l_ref)
    err_l = float((l_a[:, rows].cpu()[finite] - l_ref[finite]).abs().max())
    assert err_o <= 2e-2 and err_l <= 1e-3, (err_o, err_l)


def test_sorted_rows_skip_the_pass_and_match_it():
    """Rows already ascending (what sfa_indexer_topk writes): the forward with
    and without SFA_FWD_IDX_SORTED is bitwise the same (the pass rewrites
    them unchanged)."""
    _say("index sort: ascending rows with and without the flag")
    q, kv, idx = _case(1, 4096, 4096, 256, seed=3)
    bounds = torch.tensor([4096], dtype=torch.int32)
    srt = host_sorted(idx, bounds)
    scale = 1.0 / math.sqrt(576)
    dq, dkv, ds = (t.to(DEV) for t in (q, kv, srt))
    o_a, l_a = ops_amd.sfa_forward(dq, dkv, dkv[..., :512], ds, scale)
    o_b, l_b = ops_amd.sfa_forward(dq, dkv, dkv[..., :512], ds, scale, idx_sorted=True)
    torch.cuda.synchronize()
    assert torch.equal(o_a, o_b) and torch.equal(l_a, l_b)
