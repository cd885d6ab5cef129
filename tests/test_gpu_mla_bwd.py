"""GPU parity of the MLA shared-KV backward (one latent KV row per token,
d_qk 576, V = its first 512 dims, 65..128 query heads per KV head) on its MFMA
path (sfa_bwd with SFA_BWD_MERGE_KV): dQ and the gradient of the shared rows
(dK + dV on the first 512 dims, summed into one buffer as SFA.py:849-853
does) against the CPU oracle, relative-L2 <= 1e-2."""
import math
import sys

import pytest
import torch

import ops_amd
from ops_amd.workloads import make_workload
from oracle.sfa_oracle import sfa_backward as ref_backward
from oracle.sfa_oracle import sfa_forward as ref_forward

pytestmark = pytest.mark.gpu

GRAD_RL2 = 1e-2
DEV = "cuda"


def _say(msg):
    print(f"\n[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _rel_l2(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _ref_merged(q, kv, idx, out, lse, dout, scale, kv_lens=None, sink=None, dlse=None):
    """Reference dQ, dK + dV of the shared rows, dsink: the CPU oracle, or,
    with a gradient on lse (which the oracle does not take), the float32
    restatement of tests/fullgrid_ref.py (pinned to the oracle, dlse included,
    by tests/test_fullgrid_ref.py) on the GPU."""
    if dlse is not None:
        import fullgrid_ref as fr
        dq, dk, dv, ds = fr.backward(q, kv, kv[..., :512], idx, out, lse, dout, scale, kv_lens=kv_lens,
                                     sink=sink, dlse=dlse)
        dq, dk, dv = dq.cpu(), dk.cpu(), dv.cpu()
        ds = None if ds is None else ds.cpu()
    else:
        qc, kc = q.float().cpu(), kv.float().cpu()
        dq, dk, dv, ds = ref_backward(qc, kc, kc[..., :512], idx.cpu(), out.float().cpu(), lse.float().cpu(),
                                      dout.float().cpu(), scale,
                                      kv_lens=None if kv_lens is None else kv_lens.cpu(),
                                      sink=None if sink is None else sink.cpu())
    dkv = dk.clone()
    dkv[..., :512] += dv
    return dq, dkv, ds


def _run(q, kv, idx, dout, scale, kv_lens=None, sink=None, dlse=None, mode=None):
    out, lse = ops_amd.sfa_forward(q, kv, kv[..., :512], idx, scale, kv_lens=kv_lens, attn_sink=sink)
    dq, dkv, dv, ds = ops_amd.sfa_backward(q, kv, kv[..., :512], idx, out, lse, dout, scale, kv_lens=kv_lens,
                                           attn_sink=sink, dlse=dlse, merge_kv=True, dkv_mode=mode)
    torch.cuda.synchronize()
    assert dv is None
    return out, lse, dq, dkv, ds


def _inputs(B, S, H, K, seed, recent=True):
    w = make_workload("mla_prefill", device=DEV, seed=seed, B=B, S=S, Hq=H, K=K, with_dout=True)
    return w


@pytest.mark.parametrize("mode", ["auto", "atomic"])
def test_mla_bwd_mfma_matches_oracle_multichunk(mode):
    """S = 1024, top-k 2048, G = 128: about 3.4 MiB of chunk workspace per
    query, so the backward runs as four chunks; 'auto' sums the per-slot rows
    in a fixed order, 'atomic' adds them with fp32 atomics."""
    _say(f"MLA bwd MFMA B=1 S=1024 Hq=128 K=2048 (several chunks, dkv_mode={mode})")
    w = _inputs(1, 1024, 128, 2048, seed=3)
    out, lse, dq, dkv, _ = _run(w.q, w.k, w.idx, w.dout, w.scale, mode=mode)
    rdq, rdkv, _ = _ref_merged(w.q, w.k, w.idx, out, lse, w.dout, w.scale)
    e_q, e_kv = _rel_l2(dq.float().cpu(), rdq), _rel_l2(dkv.float().cpu(), rdkv)
    _say(f"  rel-L2 dq {e_q:.2e} dkv {e_kv:.2e}")
    assert e_q <= GRAD_RL2 and e_kv <= GRAD_RL2


@pytest.mark.parametrize("mode", ["auto", "atomic"])
@pytest.mark.parametrize("H", [128, 100, 72])
def test_mla_bwd_mfma_masking_sink_dlse(H, mode):
    """Padding inside and after the valid slots, ids at or past kv_lens, a
    fully masked query row, a sink and a gradient on lse; G = 100 and 72 leave
    the last head group partly empty."""
    _say(f"MLA bwd MFMA masking / kv_lens / sink / dlse B=2 S=96 Hq={H} K=200 dkv_mode={mode}")
    g = torch.Generator(device=DEV).manual_seed(11 + H)
    B, S, K = 2, 96, 200
    q = torch.randn(B, S, H, 576, device=DEV, generator=g).bfloat16()
    kv = torch.randn(B, S, 1, 576, device=DEV, generator=g).bfloat16()
    idx = torch.randint(0, S, (B, S, 1, K), device=DEV, generator=g, dtype=torch.int32)
    drop = torch.rand(B, S, 1, K, device=DEV, generator=g) < 0.25
    idx = torch.where(drop, torch.full_like(idx, -1), idx)          # interior -1
    idx[:, :, :, K - 17:] = -1                                       # trailing padding
    idx[0, 5] = -1                                                   # a fully masked row
    idx[1, 7, 0, :9] = S + 3                                         # ids beyond Skv
    kv_lens = torch.tensor([S, 61], device=DEV, dtype=torch.int32)   # ids >= 61 invalid in batch 1
    sink = torch.randn(H, device=DEV, generator=g)
    dlse = torch.randn(B, S, H, device=DEV, generator=g)
    dout = torch.randn(B, S, H, 512, device=DEV, generator=g).bfloat16()
    scale = 1.0 / math.sqrt(576)
    out, lse, dq, dkv, ds = _run(q, kv, idx, dout, scale, kv_lens=kv_lens, sink=sink, dlse=dlse, mode=mode)
    rdq, rdkv, rds = _ref_merged(q, kv, idx, out, lse, dout, scale, kv_lens=kv_lens, sink=sink, dlse=dlse)
    e_q, e_kv, e_s = _rel_l2(dq.float().cpu(), rdq), _rel_l2(dkv.float().cpu(), rdkv), _rel_l2(ds.cpu(), rds)
    _say(f"  rel-L2 dq {e_q:.2e} dkv {e_kv:.2e} dsink {e_s:.2e}")
    assert e_q <= GRAD_RL2 and e_kv <= GRAD_RL2 and e_s <= GRAD_RL2
    assert torch.all(dq[0, 5] == 0), "a query with no valid slot has dQ = 0"
    assert torch.all(dkv[1, 61:] == 0), "rows past kv_lens get no gradient"


def test_mla_bwd_invariant_to_invalid_encoding_and_deterministic():
    """Deterministic mode: bitwise identical results when only the encoding of
    the invalid slots changes (-1 vs ids >= Skv) and from run to run; with
    atomics dQ is still bitwise identical and dK + dV equal up to the order
    of the fp32 adds."""
    _say("MLA bwd MFMA invariance to invalid-slot encoding, determinism")
    w = _inputs(1, 256, 128, 256, seed=7)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    idx2 = torch.where(w.idx < 0, torch.full_like(w.idx, 1 << 20), w.idx)
    bwd = lambda i, m: ops_amd.sfa_backward(w.q, w.k, w.v, i, out, lse, w.dout, w.scale, merge_kv=True,
                                             dkv_mode=m)
    dq1, dkv1, _, _ = bwd(w.idx, "csr")
    dq2, dkv2, _, _ = bwd(idx2, "csr")
    dq3, dkv3, _, _ = bwd(w.idx, "csr")
    dq4, dkv4, _, _ = bwd(idx2, "atomic")
    torch.cuda.synchronize()
    assert torch.equal(dq1, dq2) and torch.equal(dkv1, dkv2)
    assert torch.equal(dq1, dq3) and torch.equal(dkv1, dkv3)
    assert torch.equal(dq1, dq4)
    # (the deterministic mode rounds each slot's row to bf16 before its fp32
    # sum, the atomic mode adds fp32 rows: both sit within ~3e-3 of the oracle)
    assert _rel_l2(dkv1.float(), dkv4.float()) <= GRAD_RL2


def test_mla_bwd_concurrent_calls_on_two_streams():
    """Two host threads run the deterministic backward (2304 queries: three
    chunks, so each call forks its reductions and the index maps of its third
    chunk onto the library's second stream) at once, each on its own torch
    stream with its own inputs. The library enqueues one such call at a time
    per device, and each call orders its work on the shared second stream
    with its own events: both results are bitwise those of the same calls
    made one after the other."""
    import threading
    _say("MLA bwd: two concurrent calls on two streams, three chunks each")
    ws = [_inputs(1, 2304, 128, 256, seed=s) for s in (31, 32)]
    fwd = [ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale) for w in ws]

    def bwd(i):
        w, (out, lse) = ws[i], fwd[i]
        return ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale, merge_kv=True)

    seq = [bwd(i) for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    got = [None, None]
    errs = []

    def run(i):
        try:
            with torch.cuda.stream(streams[i]):
                for _ in range(3):
                    got[i] = bwd(i)
            streams[i].synchronize()
        except Exception as e:  # reported below
            errs.append(e)

    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    th = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=120)
    assert not errs, errs
    assert all(not t.is_alive() for t in th)
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(got[i][0], seq[i][0]) and torch.equal(got[i][1], seq[i][1]), i


def test_mla_bwd_repeated_keys():
    """Index rows that select the same key more than once: every slot counts
    (the oracle sums each slot, SFA.py:386-467); the deterministic mode sends
    the repeats through fp32 atomics."""
    _say("MLA bwd MFMA repeated keys B=1 S=64 Hq=128 K=96")
    g = torch.Generator(device=DEV).manual_seed(21)
    B, S, H, K = 1, 64, 128, 96
    q = torch.randn(B, S, H, 576, device=DEV, generator=g).bfloat16()
    kv = torch.randn(B, S, 1, 576, device=DEV, generator=g).bfloat16()
    idx = torch.randint(0, 16, (B, S, 1, K), device=DEV, generator=g, dtype=torch.int32)  # many repeats
    dout = torch.randn(B, S, H, 512, device=DEV, generator=g).bfloat16()
    scale = 1.0 / math.sqrt(576)
    out, lse, dq, dkv, _ = _run(q, kv, idx, dout, scale)
    rdq, rdkv, _ = _ref_merged(q, kv, idx, out, lse, dout, scale)
    e_q, e_kv = _rel_l2(dq.float().cpu(), rdq), _rel_l2(dkv.float().cpu(), rdkv)
    _say(f"  rel-L2 dq {e_q:.2e} dkv {e_kv:.2e}")
    assert e_q <= GRAD_RL2 and e_kv <= GRAD_RL2


def test_mla_bwd_separate_dk_dv_generic():
    """Without the merge flag the MLA shape still returns separate dK and dV
    (generic kernels): dK + dV equals the merged MFMA result."""
    _say("MLA bwd separate dK / dV (generic) vs merged (MFMA) S=48 K=24")
    w = _inputs(1, 48, 128, 24, seed=9)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    dq_s, dk_s, dv_s, _ = ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale)
    dq_m, dkv_m, _, _ = ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale, merge_kv=True)
    torch.cuda.synchronize()
    merged = dk_s.float().clone()
    merged[..., :512] += dv_s.float()
    assert _rel_l2(dq_m.float(), dq_s.float()) <= GRAD_RL2
    assert _rel_l2(dkv_m.float(), merged) <= GRAD_RL2


def test_autograd_merges_only_views_autograd_tracks():
    """The autograd Function returns dK + dV as k's gradient only when v is
    a view of k that autograd tracks.  An alias autograd does not see (a
    detached prefix view, or a view of a second leaf over the same storage)
    shares memory but not gradients: k then gets dK alone and v's own leaf
    dV (the unmerged path), against the CPU oracle."""
    _say("MLA autograd: detached / second-leaf aliases of v vs an autograd view")
    w = _inputs(1, 48, 128, 24, seed=13)
    qc, kc = w.q.float().cpu(), w.k.float().cpu()
    out_ref, lse_ref = ref_forward(qc, kc, kc[..., :512], w.idx.cpu(), w.scale)
    rdq, rdk, rdv, _ = ref_backward(qc, kc, kc[..., :512], w.idx.cpu(), out_ref, lse_ref, w.dout.float().cpu(),
                                    w.scale)
    merged = rdk.clone()
    merged[..., :512] += rdv

    def run(make_v):
        q = w.q.clone().requires_grad_(True)
        kv = w.k.clone().requires_grad_(True)
        v, v_leaf = make_v(kv)
        out, _ = ops_amd.sparse_flash_attention(q, kv, v, w.idx, w.scale)
        (out.float() * w.dout.float()).sum().backward()
        torch.cuda.synchronize()
        return q.grad, kv.grad, (v_leaf.grad if v_leaf is not None else None)

    # an autograd view: k's gradient is dK + dV
    dq, dkv, _ = run(lambda kv: (kv[..., :512], None))
    assert _rel_l2(dq.float().cpu(), rdq) <= GRAD_RL2
    assert _rel_l2(dkv.float().cpu(), merged) <= GRAD_RL2
    # a detached alias: dK alone
    dq, dk, _ = run(lambda kv: (kv[..., :512].detach(), None))
    assert _rel_l2(dq.float().cpu(), rdq) <= GRAD_RL2
    assert _rel_l2(dk.float().cpu(), rdk) <= GRAD_RL2
    # a view of a second leaf over the same storage: dK to k, dV to that leaf
    def second_leaf(kv):
        other = kv.detach().requires_grad_(True)
        return other[..., :512], other

    dq, dk, dother = run(second_leaf)
    assert _rel_l2(dk.float().cpu(), rdk) <= GRAD_RL2
    assert dother is not None and _rel_l2(dother[..., :512].float().cpu(), rdv) <= GRAD_RL2
    assert bool((dother[..., 512:] == 0).all())
