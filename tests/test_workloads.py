"""Structure of the seeded synthetic workloads (small shapes, CPU)."""
import torch

from ops_amd.workloads import make_workload


def _check_rows(idx, allowed_hi, n_valid):
    """Valid entries first (no duplicates, in [0, allowed_hi[row]]), then -1."""
    for r in range(idx.shape[0]):
        row = idx[r]
        nv = int(n_valid[r])
        assert torch.all(row[:nv] >= 0) and torch.all(row[nv:] == -1)
        assert torch.all(row[:nv] <= allowed_hi[r])
        assert row[:nv].unique().numel() == nv


def test_tiny_structure():
    w = make_workload("tiny", S=40, K=16)
    assert w.q.dtype == torch.float32 and w.idx.dtype == torch.int32
    t = torch.arange(40)
    _check_rows(w.idx[0, :, 0], t, torch.clamp(t + 1, max=16))
    assert w.dout is not None and w.dout.shape == (1, 40, 4, 64)


def test_prefill_window_and_random_part():
    w = make_workload("prefill", S=200, K=64, Hq=4)
    idx = w.idx[0, :, 0]
    t = torch.arange(200)
    _check_rows(idx, t, torch.clamp(t + 1, max=64))
    window = 64 // 8
    for r in (0, 5, 7, 100, 199):
        row = set(idx[r][idx[r] >= 0].tolist())
        assert set(range(max(0, r - window + 1), r + 1)) <= row
    assert w.q.dtype == torch.bfloat16


def test_train_gqa_hot_share():
    w = make_workload("train_gqa", S=512, K=64, B=1, Hq=4, Hkv=2, Dqk=16, Dv=16)
    t = torch.arange(512)
    for g in range(2):
        _check_rows(w.idx[0, :, g], t, torch.clamp(t + 1, max=64))
    for share in w.meta["hot_share"]:
        assert 0.36 <= share <= 0.44, w.meta


def test_mla_prefill_recency():
    w = make_workload("mla_prefill", S=300, K=64, Hq=8, Dqk=48, Dv=32)
    assert w.v.data_ptr() == w.k.data_ptr() and w.v.shape[-1] == 32
    idx = w.idx[0, :, 0]
    t = torch.arange(300)
    _check_rows(idx, t, torch.clamp(t + 1, max=64))
    n_recent, win = 64 // 8, 64 // 2
    for r in range(64, 300, 37):
        row = idx[r]
        assert int(((row > r - win) & (row <= r)).sum()) >= n_recent


def test_mla_decode_lengths():
    w = make_workload("mla_decode", B=4, Skv=4096, K=128, Hq=8, Dqk=48, Dv=32, ctx_lo=1024)
    assert w.kv_lens is not None
    for b in range(4):
        n = int(w.kv_lens[b])
        assert 1024 <= n <= 4096
        row = w.idx[b, 0, 0]
        assert torch.all((row >= 0) & (row < n)) and row.unique().numel() == 128


def test_determinism():
    a = make_workload("prefill", S=64, K=16, Hq=2)
    b = make_workload("prefill", S=64, K=16, Hq=2)
    assert torch.equal(a.idx, b.idx) and torch.equal(a.q, b.q)
