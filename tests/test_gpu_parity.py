"""GPU parity: the HIP kernels (through libsfa's C ABI) against the CPU oracle
on identical seeded inputs.

Bars (from the task): O max-abs <= 2e-2, LSE abs <= 1e-3, dQ/dK/dV
relative-L2 <= 1e-2; index handling exact (bitwise-identical results when
only invalid entries change)."""
import ctypes
import math
import sys

import pytest
import torch

import ops_amd
from ops_amd import sfa
from ops_amd.workloads import make_workload
from oracle.sfa_oracle import sfa_backward as ref_backward
from oracle.sfa_oracle import sfa_forward as ref_forward

pytestmark = pytest.mark.gpu

O_TOL = 2e-2
LSE_TOL = 1e-3
GRAD_RL2 = 1e-2
DEV = "cuda"


def _say(msg):
    print(f"\n[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _rel_l2(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _check_fwd(out, lse, o_ref, l_ref, rows=None):
    out = out.float().cpu()
    lse = lse.float().cpu()
    if rows is not None:
        out, lse = out[:, rows], lse[:, rows]
        o_ref, l_ref = o_ref[:, rows], l_ref[:, rows]
    fin = torch.isfinite(l_ref)
    assert torch.equal(torch.isfinite(lse), fin), "LSE finiteness differs"
    assert torch.all(lse[~fin] == -math.inf)
    err_o = float((out - o_ref.float()).abs().max())
    err_l = float((lse[fin] - l_ref[fin].float()).abs().max()) if fin.any() else 0.0
    assert err_o <= O_TOL, f"O max-abs {err_o}"
    assert err_l <= LSE_TOL, f"LSE max-abs {err_l}"
    return err_o, err_l


_CACHE = {}


def _workload(name, **kw):
    """make_workload on the GPU, cached across tests (the decode KV cache is 4.8 GB)."""
    key = (name, tuple(sorted(kw.items())))
    if key not in _CACHE:
        if len(_CACHE) >= 3:
            _CACHE.pop(next(iter(_CACHE)))
        _CACHE[key] = make_workload(name, device=DEV, **kw)
    return _CACHE[key]


def _cpu(w):
    return (w.q.cpu(), w.k.cpu(), w.v.cpu(), w.idx.cpu(), None if w.kv_lens is None else w.kv_lens.cpu())


# ---------------------------------------------------------------- forward


def test_tiny_fp32_fwd_bwd():
    _say("tiny fp32 B=1 S=256 Hq=4 Hkv=1 d=64 K=64 (generic fp32 kernels)")
    w = make_workload("tiny", device=DEV)
    q, k, v, idx, _ = _cpu(w)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    o_ref, l_ref = ref_forward(q, k, v, idx, w.scale)
    _check_fwd(out, lse, o_ref, l_ref)
    dq, dk, dv, _ = ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale)
    torch.cuda.synchronize()
    g_ref = ref_backward(q, k, v, idx, out.cpu(), lse.cpu(), w.dout.cpu(), w.scale)
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), g_ref[:3]):
        assert _rel_l2(a.cpu(), b) <= GRAD_RL2, name


@pytest.mark.parametrize("S,K", [(256, 64), (1024, 256), (4096, 512), (2048, 1536)])
def test_prefill_mqa_d128(S, K):
    """(K = 1536 exceeds the d=128 kernel's 1024-slot index window: the
    library splits the top-k set and merges the splits.)"""
    _say(f"prefill bf16 MQA G=16 d=128 S={S} K={K} (d=128 kernel)")
    w = make_workload("prefill", device=DEV, S=S, K=K)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    o_ref, l_ref = ref_forward(*_cpu(w)[:4], w.scale)
    _check_fwd(out, lse, o_ref, l_ref)


@pytest.mark.parametrize("G", [1, 2, 4, 8, 16])
def test_d128_group_sizes_splits_kvlens_sink(G):
    """The d=128 kernel for every group size it serves: 2 KV heads, 96 slots
    (3 key tiles: an odd count), indices anywhere in [0, Skv) with -1 and
    out-of-range entries, per-batch kv_lens, a sink, and forced split-k."""
    _say(f"d=128 forward G={G} Hkv=2 B=2 S=40 Skv=300 K=96, splits 0/2/3")
    g = torch.Generator(device="cpu").manual_seed(100 + G)
    B, S, Skv, Hkv, K = 2, 40, 300, 2, 96
    Hq = G * Hkv
    q = torch.randn(B, S, Hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Skv, Hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Skv, Hkv, 128, generator=g).to(torch.bfloat16)
    idx = torch.randint(-40, Skv + 40, (B, S, Hkv, K), generator=g, dtype=torch.int32)
    idx[0, 3] = -1  # a fully masked row
    kv_lens = torch.tensor([300, 211], dtype=torch.int32)
    sink = torch.linspace(-1.0, 2.0, Hq)
    o_ref, l_ref = ref_forward(q, k, v, idx, 1.0 / math.sqrt(128), kv_lens=kv_lens, sink=sink)
    for ns in (0, 2, 3):
        out, lse = ops_amd.sfa_forward(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), None, kv_lens=kv_lens.to(DEV),
                                       attn_sink=sink.to(DEV), num_splits=ns)
        _check_fwd(out, lse, o_ref, l_ref)


def test_train_gqa_fwd_full():
    _say("train_gqa bf16 B=2 S=8192 Hq=32 Hkv=2 d=128 K=1024 forward")
    w = _workload("train_gqa")
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    q, k, v, idx, _ = _cpu(w)
    rows = torch.arange(0, 8192, 61)
    o_ref, l_ref = ref_forward(q, k, v, idx, w.scale,
                               query_chunks=[(b, int(r), int(r) + 1) for b in range(2) for r in rows])
    _check_fwd(out, lse, o_ref, l_ref, rows=rows)


@pytest.mark.parametrize("mode", ["csr", "atomic"])
def test_train_gqa_bwd_reduced(mode):
    """GQA fwd + bwd at S=1024, K=128 against the oracle, with both dK/dV
    schemes: 'csr' (key-major kernel + register-direct dQ kernel) and
    'atomic' (bwd_mfma_kernel: dQ and fp32-atomic dK/dV in one pass)."""
    _say(f"train_gqa bf16 B=2 S=1024 Hq=32 Hkv=2 d=128 K=128 fwd+bwd dkv_mode={mode}")
    w = make_workload("train_gqa", device=DEV, S=1024, K=128)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    q, k, v, idx, _ = _cpu(w)
    o_ref, l_ref = ref_forward(q, k, v, idx, w.scale)
    _check_fwd(out, lse, o_ref, l_ref)
    dq, dk, dv, _ = ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale, dkv_mode=mode)
    g_ref = ref_backward(q, k, v, idx, out.cpu(), lse.cpu(), w.dout.cpu(), w.scale)
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), g_ref[:3]):
        e = _rel_l2(a.cpu(), b)
        assert e <= GRAD_RL2, f"{name} rel-L2 {e}"


def test_train_gqa_bwd_full():
    """Full-size GQA backward with both dK/dV schemes (the default
    deterministic one and the fp32-atomic bwd_mfma_kernel); the oracle checks
    one (batch, kv-head) slice, which is an independent problem of its own."""
    w = _workload("train_gqa")
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    torch.cuda.synchronize()
    b, g, G = 1, 1, 16
    hs = slice(g * G, (g + 1) * G)
    q = w.q[b:b + 1, :, hs].cpu()
    k = w.k[b:b + 1, :, g:g + 1].cpu()
    v = w.v[b:b + 1, :, g:g + 1].cpu()
    idx = w.idx[b:b + 1, :, g:g + 1].cpu()
    o_s, l_s, do_s = out[b:b + 1, :, hs].cpu(), lse[b:b + 1, :, hs].cpu(), w.dout[b:b + 1, :, hs].cpu()
    g_ref = ref_backward(q, k, v, idx, o_s, l_s, do_s, w.scale)
    for mode in ("csr", "atomic"):
        _say(f"train_gqa bf16 B=2 S=8192 Hq=32 Hkv=2 d=128 K=1024 bwd dkv_mode={mode}")
        dq, dk, dv, _ = ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale, dkv_mode=mode)
        for name, a, ref in (("dq", dq[b:b + 1, :, hs], g_ref[0]), ("dk", dk[b:b + 1, :, g:g + 1], g_ref[1]),
                             ("dv", dv[b:b + 1, :, g:g + 1], g_ref[2])):
            e = _rel_l2(a.cpu(), ref)
            assert e <= GRAD_RL2, f"{mode} {name} rel-L2 {e}"
        del dq, dk, dv


@pytest.mark.parametrize("D", [64, 256])
def test_generic_bf16_bwd_large_group(D):
    """Head dims other than 128 (and the MLA 576 / 512) have no MFMA backward
    variant: at G = 32 the generic bf16 kernels run (d = 64: the per-element
    δ kernel; d = 256: the 16-byte δ kernel)."""
    _say(f"bf16 bwd G=32 d={D} (generic kernels)")
    w = make_workload("train_gqa", device=DEV, S=256, K=64, Hq=64, Hkv=2, Dqk=D, Dv=D)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    q, k, v, idx, _ = _cpu(w)
    o_ref, l_ref = ref_forward(q, k, v, idx, w.scale)
    _check_fwd(out, lse, o_ref, l_ref)
    dq, dk, dv, _ = ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale)
    g_ref = ref_backward(q, k, v, idx, out.cpu(), lse.cpu(), w.dout.cpu(), w.scale)
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), g_ref[:3]):
        e = _rel_l2(a.cpu(), b)
        assert e <= GRAD_RL2, f"{name} rel-L2 {e}"


def _bwd_with_dlse_ref(q, k, v, idx, dout, dlse, scale, kv_lens, sink):
    """Oracle gradients when a gradient dlse also reaches the returned LSE:
    d(lse)/d(s_j) = P_j, so dlse adds P·dlse to dS = P(dP - δ), i.e. δ
    becomes Σ O·dO - dlse (and dsink gains e^(sink - lse)·dlse).  Computed
    through the oracle's autograd restatement (fp64), which differentiates
    the forward directly and does not use that identity."""
    from oracle.sfa_oracle import sfa_forward_autograd
    qc, kc, vc = (t.detach().cpu().double().requires_grad_(True) for t in (q, k, v))
    sc = sink.detach().cpu().double().requires_grad_(True) if sink is not None else None
    o2, l2 = sfa_forward_autograd(qc, kc, vc, idx.cpu(), scale=scale,
                                  kv_lens=None if kv_lens is None else kv_lens.cpu(), sink=sc)
    l2f = torch.where(torch.isfinite(l2), l2, torch.zeros_like(l2))
    ((o2 * dout.cpu().double()).sum() + (l2f * dlse.cpu().double()).sum()).backward()
    return qc.grad, kc.grad, vc.grad, (sc.grad if sc is not None else None)


@pytest.mark.parametrize("mode", ["csr", "atomic"])
def test_bwd_mfma_masking_and_sink(mode):
    """d=128 backward with interior padding, kv_lens, a fully masked row,
    G = 8, an attention sink and a gradient into LSE, for both dK/dV schemes
    ('atomic' runs bwd_mfma_kernel, 'csr' the key-major + dQ kernels)."""
    _say(f"MFMA bwd: padding / kv_lens / masked row / G=8 / sink / dlse, dkv_mode={mode}")
    w = make_workload("train_gqa", device=DEV, S=512, K=128, B=1, Hq=16, Hkv=2)
    idx = w.idx.clone()
    r = torch.rand(idx.shape, generator=torch.Generator(device=DEV).manual_seed(3), device=DEV)
    idx = torch.where(r < 0.1, torch.full_like(idx, -1), idx)
    idx[:, 7] = -1
    kv_lens = torch.tensor([480], dtype=torch.int32, device=DEV)
    sink = torch.linspace(-1, 2, 16, device=DEV)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, idx, w.scale, kv_lens=kv_lens, attn_sink=sink)
    dq, dk, dv, ds = ops_amd.sfa_backward(w.q, w.k, w.v, idx, out, lse, w.dout, w.scale, kv_lens=kv_lens,
                                          attn_sink=sink, dkv_mode=mode)
    q, k, v, _, _ = _cpu(w)
    g_ref = ref_backward(q, k, v, idx.cpu(), out.cpu(), lse.cpu(), w.dout.cpu(), w.scale, kv_lens=kv_lens.cpu(),
                         sink=sink.cpu())
    for name, a, b in zip(("dq", "dk", "dv", "dsink"), (dq, dk, dv, ds), g_ref):
        e = _rel_l2(a.cpu(), b)
        assert e <= GRAD_RL2, f"{name} rel-L2 {e}"
    # the fully masked row still gets dQ = 0 (its only probability mass is the sink)
    assert torch.all(dq[:, 7] == 0)
    # unreferenced key rows (beyond kv_lens) get exactly zero dK / dV
    assert torch.all(dk[:, 480:] == 0) and torch.all(dv[:, 480:] == 0)
    # a gradient reaching LSE (autograd-derived oracle, fp64)
    dlse = torch.randn(lse.shape, generator=torch.Generator(device=DEV).manual_seed(9), device=DEV)
    dq, dk, dv, ds = ops_amd.sfa_backward(w.q, w.k, w.v, idx, out, lse, w.dout, w.scale, kv_lens=kv_lens,
                                          attn_sink=sink, dlse=dlse, dkv_mode=mode)
    g_ref = _bwd_with_dlse_ref(w.q.float(), w.k.float(), w.v.float(), idx, w.dout.float(), dlse, w.scale, kv_lens,
                               sink)
    for name, a, b in zip(("dq", "dk", "dv", "dsink"), (dq, dk, dv, ds), g_ref):
        e = _rel_l2(a.cpu(), b)
        assert e <= GRAD_RL2, f"dlse {name} rel-L2 {e}"


@pytest.mark.parametrize("G", [3, 12])
@pytest.mark.parametrize("mode", ["auto", "atomic"])
def test_d128_non_power_of_two_groups(G, mode):
    """d=128 forward and backward at group sizes that are not powers of two
    (the deterministic scheme needs one, so 'auto' takes the atomic
    bwd_mfma_kernel too), with interior padding, out-of-range ids, kv_lens,
    a fully masked row, a sink and a gradient into LSE."""
    _say(f"d=128 G={G} Hkv=2 B=2 S=96 Skv=160 K=64 fwd+bwd, dkv_mode={mode}")
    g = torch.Generator(device="cpu").manual_seed(200 + G)
    B, S, Skv, Hkv, K = 2, 96, 160, 2, 64
    Hq = G * Hkv
    q = torch.randn(B, S, Hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Skv, Hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Skv, Hkv, 128, generator=g).to(torch.bfloat16)
    dout = torch.randn(B, S, Hq, 128, generator=g).to(torch.bfloat16)
    idx = torch.randint(-20, Skv + 20, (B, S, Hkv, K), generator=g, dtype=torch.int32)
    idx[1, 5] = -1  # a fully masked row
    kv_lens = torch.tensor([160, 117], dtype=torch.int32)
    sink = torch.linspace(-1.0, 2.0, Hq)
    dlse = torch.randn(B, S, Hq, generator=g)
    scale = 1.0 / math.sqrt(128)
    o_ref, l_ref = ref_forward(q, k, v, idx, scale, kv_lens=kv_lens, sink=sink)
    qd, kd, vd, idd, kld, sd = (t.to(DEV) for t in (q, k, v, idx, kv_lens, sink))
    out, lse = ops_amd.sfa_forward(qd, kd, vd, idd, scale, kv_lens=kld, attn_sink=sd)
    _check_fwd(out, lse, o_ref, l_ref)
    dq, dk, dv, ds = ops_amd.sfa_backward(qd, kd, vd, idd, out, lse, dout.to(DEV), scale, kv_lens=kld,
                                          attn_sink=sd, dlse=dlse.to(DEV), dkv_mode=mode)
    g_ref = _bwd_with_dlse_ref(q.float(), k.float(), v.float(), idx, dout.float(), dlse, scale, kv_lens, sink)
    for name, a, b in zip(("dq", "dk", "dv", "dsink"), (dq, dk, dv, ds), g_ref):
        e = _rel_l2(a.cpu(), b)
        assert e <= GRAD_RL2, f"{name} rel-L2 {e}"


@pytest.mark.parametrize("G,Hkv,mode", [(32, 1, "auto"), (32, 2, "atomic"), (64, 1, "auto"), (64, 1, "csr"),
                                         (64, 1, "atomic"), (48, 1, "auto"), (128, 1, "csr"), (20, 1, "auto"),
                                         (40, 2, "atomic"), (100, 1, "auto")])
def test_d128_large_groups(G, Hkv, mode):
    """d=128 with more than 16 query heads per KV head, the reference's own
    shape class (one shared kv, query heads tiled by 32, SFA.py:35-48, 88):
    the MFMA kernels split the heads into groups of 16.  Forward and backward
    with interior padding, ids past Skv and past kv_lens, a fully masked row,
    a sink and a gradient into LSE; S = 320 spans several key blocks and, at
    G = 64, several 128-query-block chunks of the deterministic scheme (G = 48
    is not a power of two: 'auto' then takes the atomic scheme).  G = 20, 40
    and 100 leave the last head group partly empty, and at G = 100 the
    shared-tile kernels' eighth wave has no head at all (heads 112-127): it
    still loads its share of every tile and joins every barrier."""
    _say(f"d=128 G={G} Hkv={Hkv} B=2 S=320 Skv=384 K=96 fwd+bwd, dkv_mode={mode}")
    g = torch.Generator(device="cpu").manual_seed(300 + G + Hkv)
    B, S, Skv, K = 2, 320, 384, 96
    Hq = G * Hkv
    q = torch.randn(B, S, Hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Skv, Hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Skv, Hkv, 128, generator=g).to(torch.bfloat16)
    dout = torch.randn(B, S, Hq, 128, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(Skv + 40, generator=g)[:K] - 20 for _ in range(B * S * Hkv)])
    idx = idx.view(B, S, Hkv, K).to(torch.int32)
    idx[:, :, :, K - 9:] = -1   # trailing padding
    idx[1, 5] = -1              # a fully masked row
    kv_lens = torch.tensor([Skv, 301], dtype=torch.int32)
    sink = torch.linspace(-1.0, 2.0, Hq)
    dlse = torch.randn(B, S, Hq, generator=g)
    scale = 1.0 / math.sqrt(128)
    o_ref, l_ref = ref_forward(q, k, v, idx, scale, kv_lens=kv_lens, sink=sink)
    qd, kd, vd, idd, kld, sd = (t.to(DEV) for t in (q, k, v, idx, kv_lens, sink))
    out, lse = ops_amd.sfa_forward(qd, kd, vd, idd, scale, kv_lens=kld, attn_sink=sd)
    _check_fwd(out, lse, o_ref, l_ref)
    dq, dk, dv, ds = ops_amd.sfa_backward(qd, kd, vd, idd, out, lse, dout.to(DEV), scale, kv_lens=kld,
                                          attn_sink=sd, dlse=dlse.to(DEV), dkv_mode=mode)
    g_ref = _bwd_with_dlse_ref(q.float(), k.float(), v.float(), idx, dout.float(), dlse, scale, kv_lens, sink)
    for name, a, b in zip(("dq", "dk", "dv", "dsink"), (dq, dk, dv, ds), g_ref):
        e = _rel_l2(a.cpu(), b)
        assert e <= GRAD_RL2, f"{name} rel-L2 {e}"
    assert torch.all(dq[1, 5] == 0)
    assert torch.all(dk[1, 301:] == 0) and torch.all(dv[1, 301:] == 0)


def test_d128_large_group_decode_splits():
    """Decode with G = 64 (one shared kv, 4 head groups of 16 per sequence
    and split-k over the top-k set): against the oracle at 1, 2 and 4
    splits, with kv_lens and a sink."""
    _say("d=128 decode G=64 B=4 Skv=4096 K=1024, splits 1/2/4")
    g = torch.Generator(device="cpu").manual_seed(77)
    B, Skv, H, K = 4, 4096, 64, 1024
    q = torch.randn(B, 1, H, 128, generator=g).to(torch.bfloat16)
    kv = torch.randn(B, Skv, 1, 128, generator=g).to(torch.bfloat16)
    kv_lens = torch.tensor([4096, 3000, 1500, 700], dtype=torch.int32)
    idx = torch.stack([torch.randperm(int(n), generator=g)[:K] if n >= K else
                       torch.cat([torch.randperm(int(n), generator=g), torch.full((K - int(n),), -1)])
                       for n in kv_lens]).view(B, 1, 1, K).to(torch.int32)
    sink = torch.linspace(-0.5, 1.0, H)
    scale = 1.0 / math.sqrt(128)
    o_ref, l_ref = ref_forward(q, kv, kv, idx, scale, kv_lens=kv_lens, sink=sink)
    qd, kd, idd, kld, sd = (t.to(DEV) for t in (q, kv, idx, kv_lens, sink))
    for splits in (1, 2, 4):
        out, lse = ops_amd.sfa_forward(qd, kd, kd, idd, scale, kv_lens=kld, attn_sink=sd, num_splits=splits)
        _check_fwd(out, lse, o_ref, l_ref)


@pytest.mark.parametrize("S,K", [(300, 64), (1024, 256)])
def test_mla_prefill_reduced(S, K):
    _say(f"mla_prefill bf16 Hq=128 d_qk=576 d_v=512 S={S} K={K} (MFMA T=32 path)")
    w = make_workload("mla_prefill", device=DEV, S=S, K=K)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    o_ref, l_ref = ref_forward(*_cpu(w)[:4], w.scale)
    _check_fwd(out, lse, o_ref, l_ref)


@pytest.mark.parametrize("Hq", [80, 96, 112])
def test_mla_prefill_partial_head_slices(Hq):
    """G = Hq not a multiple of the 32-head slice: the last slices hold absent
    heads, whose lanes still take part in the staged row stores; with a sink."""
    _say(f"mla_prefill bf16 Hq={Hq} d_qk=576 d_v=512 S=200 K=64 with sink")
    w = make_workload("mla_prefill", device=DEV, S=200, K=64, Hq=Hq)
    sink = torch.randn(Hq, generator=torch.Generator().manual_seed(3)).to(DEV)
    out = torch.full(w.q.shape[:3] + (512,), float("nan"), dtype=w.q.dtype, device=DEV)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, attn_sink=sink, out=out)
    o_ref, l_ref = ref_forward(*_cpu(w)[:4], w.scale, sink=sink.cpu())
    _check_fwd(out, lse, o_ref, l_ref)


def test_mla_prefill_full_sampled():
    _say("mla_prefill bf16 full S=32768 K=2048 Hq=128 (sampled rows vs oracle)")
    w = make_workload("mla_prefill", device=DEV)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 100, 2047, 2048, 5000, 16383, 30000, 32767])
    q = w.q[:, rows].cpu()
    idx = w.idx[:, rows].cpu()
    o_ref, l_ref = ref_forward(q, w.k.cpu(), w.v.cpu(), idx, w.scale)
    _check_fwd(out[:, rows], lse[:, rows], o_ref, l_ref)


def test_mla_prefill_persistent_schedule():
    """S = 4100 queries (>= 4096 work items: one workgroup per CU claims them
    from per-XCD counters; 4100 is not a multiple of 8 or 256, so the XCD
    queues differ in length and the plain item mapping is used), with fully
    masked rows and rows whose valid slots end early: sampled rows match the
    oracle, and a second run is bitwise identical (the claim order varies, a
    row's arithmetic does not)."""
    _say("mla_prefill bf16 persistent S=4100 K=256 Hq=128 (sampled rows vs oracle, run-to-run bitwise)")
    w = make_workload("mla_prefill", device=DEV, S=4100, K=256)
    idx = w.idx.clone()
    idx[:, 4000] = -1                 # no valid slot
    idx[:, 4001, :, 40:] = -1         # valid slots end in the second tile
    out1, lse1 = ops_amd.sfa_forward(w.q, w.k, w.v, idx, w.scale)
    out2, lse2 = ops_amd.sfa_forward(w.q, w.k, w.v, idx, w.scale)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2) and torch.equal(lse1, lse2)
    assert torch.all(out1[:, 4000] == 0) and torch.all(lse1[:, 4000] == float("-inf"))
    rows = torch.tensor([0, 1, 255, 256, 1000, 2047, 3333, 4001, 4095, 4096, 4099])
    o_ref, l_ref = ref_forward(w.q[:, rows].cpu(), w.k.cpu(), w.v.cpu(), idx[:, rows].cpu(), w.scale)
    _check_fwd(out1[:, rows], lse1[:, rows], o_ref, l_ref)


@pytest.mark.parametrize("Hq,Hkv,S", [(80, 1, 4100), (112, 1, 4100), (256, 2, 2050)])
def test_mla_prefill_persistent_head_slices_and_kv_heads(Hq, Hkv, S):
    """The persistent MLA forward (>= 4096 work items) with G = Hq / Hkv not a
    multiple of the 32-head slice (the last slices hold absent heads: the
    output rounds then wait for all their stores) or with two KV heads (work
    items over (query, kv head)), a sink, NaN-filled outputs: every row
    written, sampled rows against the oracle."""
    _say(f"mla_prefill persistent Hq={Hq} Hkv={Hkv} S={S} K=256 with sink")
    w = make_workload("mla_prefill", device=DEV, S=S, K=256, Hq=Hq, Hkv=Hkv, seed=9)
    sink = torch.linspace(-1.5, 1.5, Hq, device=DEV)
    out = torch.full(w.q.shape[:3] + (512,), float("nan"), dtype=w.q.dtype, device=DEV)
    lse = torch.full(w.q.shape[:3], float("nan"), dtype=torch.float32, device=DEV)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, attn_sink=sink, out=out, lse=lse)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all()), "an output row was not written"
    rows = torch.tensor([0, 1, 255, 1000, S // 2, S - 2, S - 1])
    o_ref, l_ref = ref_forward(w.q[:, rows].cpu(), w.k.cpu(), w.v.cpu(), w.idx[:, rows].cpu(), w.scale,
                               sink=sink.cpu())
    _check_fwd(out[:, rows], lse[:, rows], o_ref, l_ref)


def _decode_compact(w):
    """Gather the referenced rows on the GPU so the oracle sees a small KV."""
    B, K = w.idx.shape[0], w.idx.shape[3]
    rows = w.idx[:, 0, 0].long().clamp_min(0)
    kg = torch.stack([w.k[b, rows[b], 0] for b in range(B)]).unsqueeze(2)  # [B, K, 1, Dqk]
    valid = (w.idx[:, 0, 0] >= 0) & (w.idx[:, 0, 0] < w.kv_lens[:, None])
    cidx = torch.where(valid, torch.arange(K, device=w.idx.device, dtype=torch.int32)[None, :],
                       torch.full_like(w.idx[:, 0, 0], -1)).view(B, 1, 1, K)
    return kg.cpu(), cidx.cpu()


@pytest.mark.parametrize("splits", [0, 1, 2, 4, 8])
def test_mla_decode_full(splits):
    _say(f"mla_decode bf16 B=64 Skv=65536 Hq=128 K=2048 num_splits={splits}")
    w = _workload("mla_decode")
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, kv_lens=w.kv_lens, num_splits=splits)
    kg, cidx = _decode_compact(w)
    o_ref, l_ref = ref_forward(w.q.cpu(), kg, kg[..., :512], cidx, w.scale)
    _check_fwd(out, lse, o_ref, l_ref)


# ---------------------------------------------------------------- index handling


@pytest.mark.parametrize("shape", ["d128", "mla"])
def test_invalid_entries_are_exact(shape):
    """Replacing invalid entries by other invalid values (-1 anywhere, < -1,
    >= Skv, >= kv_lens) gives bitwise-identical O and LSE; a row with no
    valid slot gives O = 0, LSE = -inf."""
    _say(f"index invariants {shape}")
    if shape == "d128":
        w = make_workload("prefill", device=DEV, S=256, K=64)
    else:
        w = make_workload("mla_prefill", device=DEV, S=256, K=64)
    Skv = w.k.shape[1]
    kv_lens = torch.tensor([Skv - 7], dtype=torch.int32, device=DEV)
    idx = w.idx.clone()
    g = torch.Generator(device=DEV).manual_seed(5)
    r = torch.rand(idx.shape, generator=g, device=DEV)
    idx = torch.where(r < 0.15, torch.full_like(idx, -1), idx)  # interior padding
    idx[:, 3] = -1                                              # a fully masked row
    out0, lse0 = ops_amd.sfa_forward(w.q, w.k, w.v, idx, w.scale, kv_lens=kv_lens)
    valid = (idx >= 0) & (idx < kv_lens.view(1, 1, 1, 1))
    for bad in (-5, Skv, Skv - 3, 1 << 30):
        idx2 = torch.where(valid, idx, torch.full_like(idx, bad))
        out2, lse2 = ops_amd.sfa_forward(w.q, w.k, w.v, idx2, w.scale, kv_lens=kv_lens)
        assert torch.equal(out0, out2) and torch.equal(lse0, lse2), bad
    assert torch.all(out0[:, 3] == 0) and torch.all(torch.isneginf(lse0[:, 3]))
    o_ref, l_ref = ref_forward(w.q.cpu(), w.k.cpu(), w.v.cpu(), idx.cpu(), w.scale, kv_lens=kv_lens.cpu())
    _check_fwd(out0, lse0, o_ref, l_ref)


def test_slot_permutation_and_duplicates():
    _say("slot permutation / duplicates d128")
    w = make_workload("prefill", device=DEV, S=256, K=64)
    out0, lse0 = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    perm = torch.randperm(64, device=DEV)
    out1, lse1 = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx[..., perm].contiguous(), w.scale)
    # summation order differs, so compare each against the oracle (outputs
    # are rounded to bf16: the two runs may differ by one bf16 ulp)
    o_ref, l_ref = ref_forward(w.q.cpu(), w.k.cpu(), w.v.cpu(), w.idx.cpu(), w.scale)
    _check_fwd(out0, lse0, o_ref, l_ref)
    _check_fwd(out1, lse1, o_ref, l_ref)
    lse_diff = float((lse0 - lse1).abs().max())
    assert lse_diff <= 1e-4, lse_diff
    dup = w.idx.clone()
    dup[..., 1] = dup[..., 0]
    out2, lse2 = ops_amd.sfa_forward(w.q, w.k, w.v, dup, w.scale)
    o_ref, l_ref = ref_forward(w.q.cpu(), w.k.cpu(), w.v.cpu(), dup.cpu(), w.scale)
    _check_fwd(out2, lse2, o_ref, l_ref)


def test_sink_forward_mfma_and_generic():
    _say("attention sink (MLA MFMA and generic fp32)")
    for name, kw in (("mla_prefill", dict(S=128, K=64)), ("tiny", dict(S=64, K=16))):
        w = make_workload(name, device=DEV, **kw)
        Hq = w.q.shape[2]
        sink = torch.linspace(-2, 3, Hq, device=DEV)
        out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, attn_sink=sink)
        o_ref, l_ref = ref_forward(w.q.cpu(), w.k.cpu(), w.v.cpu(), w.idx.cpu(), w.scale, sink=sink.cpu())
        _check_fwd(out, lse, o_ref, l_ref)


def test_mla_alias_equals_contiguous_copy():
    _say("MLA v = kv[..., :512] view vs contiguous copy (generic path)")
    w = make_workload("mla_prefill", device=DEV, S=96, K=32, Hq=128)
    out0, lse0 = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    out1, lse1 = ops_amd.sfa_forward(w.q, w.k, w.v.contiguous(), w.idx, w.scale)
    o_diff = float((out0.float() - out1.float()).abs().max())
    lse_diff = float((lse0 - lse1).abs().max())
    assert o_diff <= O_TOL, o_diff
    assert lse_diff <= 1e-4, lse_diff


def test_autograd_function_and_dlse():
    _say("autograd Function with gradients into out and lse (fp32 tiny)")
    w = make_workload("tiny", device=DEV, S=48, K=16)
    q, k, v = (t.clone().requires_grad_(True) for t in (w.q, w.k, w.v))
    out, lse = ops_amd.sparse_flash_attention(q, k, v, w.idx, w.scale)
    gl = torch.randn(lse.shape, device=DEV)
    ((out * w.dout).sum() + (torch.where(torch.isfinite(lse), lse, 0) * gl).sum()).backward()
    from oracle.sfa_oracle import sfa_forward_autograd
    qc, kc, vc = (t.detach().cpu().double().requires_grad_(True) for t in (w.q, w.k, w.v))
    o2, l2 = sfa_forward_autograd(qc, kc, vc, w.idx.cpu(), scale=w.scale)
    ((o2 * w.dout.cpu().double()).sum() + (l2 * gl.cpu().double()).sum()).backward()
    for a, b in ((q, qc), (k, kc), (v, vc)):
        assert _rel_l2(a.grad.cpu(), b.grad) <= GRAD_RL2


@pytest.mark.parametrize("G,Hkv,splits,vk", [(1, 2, 0, False), (4, 1, 3, False), (16, 1, 0, True),
                                              (32, 1, 0, True), (64, 1, 2, True), (64, 1, 0, False),
                                              (48, 2, 0, False), (100, 1, 0, True), (20, 1, 4, False)])
def test_d64_forward(G, Hkv, splits, vk):
    """Head dim 64 (d_qk = d_v = 64, bf16), the width of sink-attention
    models, on the register-gather MFMA forward: G <= 16 one wave per head
    group of 16 (fwd_d128_kernel<64>), 16 < G <= 64 the shared-tile kernel
    (fwd_d128g_kernel<64>: 2 or 4 waves gathering whole 8-row load
    instructions), G > 64 head groups again.  v the same tensor as k (the
    reference's single kv) or separate rows; split-k with the generic
    combine; interior padding, ids past Skv and past kv_lens, a fully masked
    row and a sink.  Against the oracle's bars; the backward at this width
    runs the generic kernels, checked against the oracle too."""
    _say(f"d=64 G={G} Hkv={Hkv} splits={splits} v_is_k={vk} B=2 S=160 Skv=200 K=80")
    g = torch.Generator(device="cpu").manual_seed(640 + G + Hkv + splits)
    B, S, Skv, K = 2, 160, 200, 80
    Hq = G * Hkv
    q = torch.randn(B, S, Hq, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Skv, Hkv, 64, generator=g).to(torch.bfloat16)
    v = k if vk else torch.randn(B, Skv, Hkv, 64, generator=g).to(torch.bfloat16)
    dout = torch.randn(B, S, Hq, 64, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(Skv + 30, generator=g)[:K] - 15 for _ in range(B * S * Hkv)])
    idx = idx.view(B, S, Hkv, K).to(torch.int32)
    idx[:, :, :, K - 7:] = -1
    idx[1, 3] = -1
    kv_lens = torch.tensor([Skv, 151], dtype=torch.int32)
    sink = torch.linspace(-1.0, 2.0, Hq)
    scale = 1.0 / 8.0
    o_ref, l_ref = ref_forward(q, k, v, idx, scale, kv_lens=kv_lens, sink=sink)
    qd, kd, idd, kld, sd = (t.to(DEV) for t in (q, k, idx, kv_lens, sink))
    vd = kd if vk else v.to(DEV)
    out, lse = ops_amd.sfa_forward(qd, kd, vd, idd, scale, kv_lens=kld, attn_sink=sd, num_splits=splits)
    _check_fwd(out, lse, o_ref, l_ref)
    assert torch.all(out[1, 3] == 0)
    if splits == 0 and G in (16, 64):
        dq, dk, dv, ds = ops_amd.sfa_backward(qd, kd, vd, idd, out, lse, dout.to(DEV), scale, kv_lens=kld,
                                              attn_sink=sd)
        g_ref = ref_backward(q.float(), k.float(), v.float(), idx, o_ref, l_ref, dout.float(), scale,
                             kv_lens=kv_lens, sink=sink)
        for name, a, b in zip(("dq", "dk", "dv", "dsink"), (dq, dk, dv, ds), g_ref):
            e = _rel_l2(a.cpu(), b)
            assert e <= GRAD_RL2, f"{name} rel-L2 {e}"


@pytest.mark.parametrize("H,D,dtypes", [(16, 128, (torch.float32, torch.bfloat16)), (64, 128, (torch.bfloat16,)),
                                         (32, 576, (torch.bfloat16,)), (64, 64, (torch.bfloat16,)),
                                         (32, 64, (torch.bfloat16,))])
def test_reference_signature_shim(H, D, dtypes):
    """SparseFlashAttentionTriton.apply(q[S,B,H,D], kv[S_kv,B,D], sink[H],
    idx[S,B,K], scale) -> out, with grads (q, kv, sink), against the oracle
    (K = V = the whole kv row, one KV head, so out is D wide as
    torch.empty_like(q) makes it, SFA.py:104, 456), at the reference's own
    head tiling (BLOCK_H = 32 and multiples, SFA.py:35-48) and at the MLA
    row width D = 576."""
    _say(f"reference-signature SBHD shim H={H} D={D} {[str(d) for d in dtypes]}")
    for dtype in dtypes:
        g = torch.Generator(device=DEV).manual_seed(11 + H + D)
        S, B, K = 96, 2, 48
        q = torch.randn(S, B, H, D, device=DEV, generator=g).to(dtype).requires_grad_(True)
        kv = torch.randn(S, B, D, device=DEV, generator=g).to(dtype).requires_grad_(True)
        sink = torch.randn(H, device=DEV, generator=g).requires_grad_(True)
        idx = torch.randint(-1, S, (S, B, K), device=DEV, generator=g, dtype=torch.int32)
        dout = torch.randn(S, B, H, D, device=DEV, generator=g).to(dtype)
        out = ops_amd.SparseFlashAttentionTriton.apply(q, kv, sink, idx, 0.1)
        assert tuple(out.shape) == (S, B, H, D)
        # contiguous like the reference's empty_like(q) (SFA.py:104): views work
        assert out.is_contiguous() and out.view(S, B, H * D).shape == (S, B, H * D)
        out.backward(dout)
        assert q.grad.is_contiguous() and kv.grad.is_contiguous()
        qb = q.detach().permute(1, 0, 2, 3).cpu()
        kb = kv.detach().permute(1, 0, 2).unsqueeze(2).cpu()
        ib = idx.permute(1, 0, 2).unsqueeze(2).cpu()
        o_ref, l_ref = ref_forward(qb, kb, kb, ib, 0.1, sink=sink.detach().cpu())
        err = float((out.detach().permute(1, 0, 2, 3).float().cpu() - o_ref).abs().max())
        assert err <= O_TOL, (dtype, err)
        dq, dk, dv, ds = ref_backward(qb, kb, kb, ib, o_ref, l_ref, dout.permute(1, 0, 2, 3).cpu(), 0.1,
                                      sink=sink.detach().cpu())
        assert _rel_l2(q.grad.permute(1, 0, 2, 3).cpu(), dq) <= GRAD_RL2
        assert _rel_l2(kv.grad.permute(1, 0, 2).unsqueeze(2).cpu(), dk + dv) <= GRAD_RL2
        assert _rel_l2(sink.grad.cpu(), ds) <= GRAD_RL2


def test_mla_shared_kv_backward_autograd():
    """The MLA training shape (one latent KV row per token, d_qk 576, V = its
    first 512 dims, G = 128): through autograd (v a prefix view of kv, so the
    backward takes the merged MFMA path) the shared kv's gradient is dK + dV
    (the reference sums both into one buffer, SFA.py:849-853)."""
    _say("MLA shared-kv backward B=1 S=48 Hq=128 d 576/512 K=24 (autograd, merged MFMA path)")
    g = torch.Generator(device=DEV).manual_seed(5)
    B, S, H, K = 1, 48, 128, 24
    q = torch.randn(B, S, H, 576, device=DEV, generator=g).bfloat16().requires_grad_(True)
    kv = torch.randn(B, S, 1, 576, device=DEV, generator=g).bfloat16().requires_grad_(True)
    idx = torch.randint(-1, S, (B, S, 1, K), device=DEV, generator=g, dtype=torch.int32)
    sink = torch.randn(H, device=DEV, generator=g).requires_grad_(True)
    dout = torch.randn(B, S, H, 512, device=DEV, generator=g).bfloat16()
    scale = 1.0 / math.sqrt(576)
    out, lse = ops_amd.sparse_flash_attention(q, kv, kv[..., :512], idx, scale, attn_sink=sink)
    out.backward(dout)
    qc, kc = q.detach().float().cpu(), kv.detach().float().cpu()
    o_ref, l_ref = ref_forward(qc, kc, kc[..., :512], idx.cpu(), scale, sink=sink.detach().cpu())
    _check_fwd(out.detach(), lse.detach(), o_ref, l_ref)
    dq, dk, dv, ds = ref_backward(qc, kc, kc[..., :512], idx.cpu(), o_ref, l_ref, dout.float().cpu(), scale,
                                  sink=sink.detach().cpu())
    dkv = dk.clone()
    dkv[..., :512] += dv
    assert _rel_l2(q.grad.float().cpu(), dq) <= GRAD_RL2
    assert _rel_l2(kv.grad.float().cpu(), dkv) <= GRAD_RL2
    assert _rel_l2(sink.grad.cpu(), ds) <= GRAD_RL2


@pytest.mark.parametrize("splits", [2, 4, 8])
def test_mla_decode_splits_sink(splits):
    """The d_v = 512 split merge (2, 4 or 8 splits) with an attention sink and
    per-sequence kv_lens, against the oracle."""
    _say(f"mla_decode bf16 B=4 Skv=2048 Hq=128 K=512 num_splits={splits} sink")
    w = make_workload("mla_decode", device=DEV, B=4, Skv=2048, K=512, ctx_lo=300)
    sink = torch.linspace(-1.0, 2.0, w.q.shape[2], device=DEV)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, kv_lens=w.kv_lens, attn_sink=sink,
                                   num_splits=splits)
    o_ref, l_ref = ref_forward(w.q.cpu(), w.k.cpu(), w.v.cpu(), w.idx.cpu(), w.scale, kv_lens=w.kv_lens.cpu(),
                               sink=sink.cpu())
    _check_fwd(out, lse, o_ref, l_ref)


@pytest.mark.parametrize("Hq,Hkv,splits", [(100, 1, 4), (256, 2, 4), (72, 1, 2)])
def test_mla_decode_head_counts(Hq, Hkv, splits):
    """The split-k MLA decode and its merge at head counts other than 128 on
    one KV head: partly empty 32-head slices (100, 72 heads) and two KV heads
    (256 heads, work items over (sequence, kv head)), with kv_lens and a sink,
    NaN-filled outputs: every row written, against the oracle."""
    _say(f"mla_decode B=5 Skv=3000 Hq={Hq} Hkv={Hkv} K=512 splits={splits} sink")
    w = make_workload("mla_decode", device=DEV, B=5, Skv=3000, K=512, Hq=Hq, Hkv=Hkv, ctx_lo=700, seed=6)
    sink = torch.linspace(-2.0, 1.0, Hq, device=DEV)
    out = torch.full(w.q.shape[:3] + (512,), float("nan"), dtype=w.q.dtype, device=DEV)
    lse = torch.full(w.q.shape[:3], float("nan"), dtype=torch.float32, device=DEV)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, kv_lens=w.kv_lens, attn_sink=sink,
                                   num_splits=splits, out=out, lse=lse)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all()), "an output row was not written"
    o_ref, l_ref = ref_forward(w.q.cpu(), w.k.cpu(), w.v.cpu(), w.idx.cpu(), w.scale, kv_lens=w.kv_lens.cpu(),
                               sink=sink.cpu())
    _check_fwd(out, lse, o_ref, l_ref)


@pytest.mark.parametrize("splits", [2, 4, 8])
def test_mla_decode_any_workspace_contents(splits):
    """The C ABI's workspace is scratch: with a workspace pre-filled with
    random bytes, 13 sequences (an item count that is not a multiple of 8:
    the splits of one sequence run on different XCDs), then a second call on
    the same workspace: both within the oracle's bars, bitwise equal to each
    other."""
    _say(f"mla_decode B=13 Skv=4096 Hq=128 K=1024 splits={splits}, random workspace bytes")
    from ops_amd import _lib
    w = make_workload("mla_decode", device=DEV, B=13, Skv=4096, K=1024, ctx_lo=1500, seed=3)
    lib = _lib.load()
    B, _, Hq, _ = w.q.shape
    res = []
    wbuf = None
    for call in range(2):
        out = torch.full((B, 1, Hq, 512), float("nan"), dtype=w.q.dtype, device=DEV)
        lse = torch.full((B, 1, Hq), float("nan"), dtype=torch.float32, device=DEV)
        a = sfa._fwd_args(w.q, w.k, w.v, w.idx, out, lse, w.scale, w.kv_lens, None, splits)
        ws = lib.sfa_fwd_workspace_size(ctypes.byref(a))
        if wbuf is None:
            wbuf = torch.randint(0, 256, (ws,), dtype=torch.uint8, device=DEV)
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.sfa_fwd(ctypes.byref(a), ctypes.c_void_p(wbuf.data_ptr()), ws, stream))
        torch.cuda.synchronize()
        res.append((out, lse))
    o_ref, l_ref = ref_forward(w.q.cpu(), w.k.cpu(), w.v.cpu(), w.idx.cpu(), w.scale, kv_lens=w.kv_lens.cpu())
    for out, lse in res:
        _check_fwd(out, lse, o_ref, l_ref)
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
