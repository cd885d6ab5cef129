"""Host-layer behaviour that needs no GPU: validation and error mapping of
ops_amd.sfa mirror the reference's ValueError paths (SFA.py:52-53, 63-64)."""
import pytest
import torch

import ops_amd
from ops_amd import sfa


def _cpu_case(K=4):
    q = torch.randn(1, 3, 4, 8)
    k = torch.randn(1, 5, 2, 8)
    v = torch.randn(1, 5, 2, 8)
    idx = torch.zeros(1, 3, 2, K, dtype=torch.int32)
    return q, k, v, idx


def test_empty_index_raises_like_reference():
    q, k, v, idx = _cpu_case(K=0)
    with pytest.raises(ValueError, match="empty"):
        ops_amd.sparse_flash_attention(q, k, v, idx)


def test_cpu_tensors_are_rejected_not_computed():
    q, k, v, idx = _cpu_case()
    with pytest.raises(ValueError, match="GPU"):
        ops_amd.sparse_flash_attention(q, k, v, idx)


@pytest.mark.parametrize("bad", ["hq", "idxshape", "dtype", "rank"])
def test_shape_and_dtype_validation(bad):
    q, k, v, idx = _cpu_case()
    if bad == "hq":
        q = torch.randn(1, 3, 3, 8)
    elif bad == "idxshape":
        idx = torch.zeros(1, 3, 1, 4, dtype=torch.int32)
    elif bad == "dtype":
        q = q.double()
    elif bad == "rank":
        q = q[0]
    with pytest.raises(ValueError):
        sfa._validate(q, k, v, idx, None, None)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from ops_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("SFA_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(_lib.SFAError):
        _lib.load()


def test_kv_merge_only_for_views_autograd_tracks():
    """The autograd Function returns dK + dV as k's gradient (None for v)
    only where autograd itself would add v's gradient into k's rows: v is k,
    or a prefix view of k (or of k's base) that autograd tracks, and both
    want a gradient.  Same-memory aliases that autograd does not see (a
    detached view, a second leaf over one storage, a view taken under
    no_grad) keep separate gradients; so do prefixes whose memory differs."""
    kv = torch.randn(2, 6, 1, 12, requires_grad=True)
    m = sfa._merge_in_autograd
    assert m(kv, kv[..., :8], True, True)                      # MLA: v = kv[..., :512]
    assert m(kv, kv, True, True)                               # v is k
    k2 = kv.view(2, 6, 1, 12)
    assert m(k2, kv[..., :8], True, True)                      # k and v views of one base
    assert not m(kv, kv[..., :8].detach(), True, False)        # detached alias
    other = kv.detach().requires_grad_(True)
    assert not m(kv, other[..., :8], True, True)               # second leaf over the same storage
    with torch.no_grad():
        vng = kv[..., :8]
    assert not m(kv, vng, True, False)                         # view without a gradient
    assert not m(kv, kv[..., :8], True, False)                 # v's gradient not wanted
    assert not m(kv, kv[..., 4:12], True, True)                # not a prefix of the rows
    assert not m(kv, kv[:, :3, :, :8], True, True)             # fewer rows than k
