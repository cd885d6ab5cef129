"""Pins tests/fullgrid_ref.py (the float32 full-grid evaluation the GPU tests
use at full workload sizes) against the CPU oracle on small inputs, with
padding, out-of-range ids, kv_lens, a fully masked row, a sink and a gradient
into LSE; and shows that a planted mistake in it is caught."""
import math

import torch

import fullgrid_ref as fr
from oracle.sfa_oracle import sfa_backward, sfa_forward, sfa_forward_autograd


def _inputs(seed=0, B=2, S=20, Skv=33, Hq=6, Hkv=2, D=16, Dv=12, K=10):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, Hq, D, generator=g)
    k = torch.randn(B, Skv, Hkv, D, generator=g)
    v = torch.randn(B, Skv, Hkv, Dv, generator=g)
    dout = torch.randn(B, S, Hq, Dv, generator=g)
    idx = torch.randint(-5, Skv + 5, (B, S, Hkv, K), generator=g, dtype=torch.int32)
    idx[1, 4] = -1
    kv_lens = torch.tensor([Skv, 21], dtype=torch.int32)
    sink = torch.linspace(-1.0, 1.5, Hq)
    return q, k, v, dout, idx, kv_lens, sink


def test_forward_matches_oracle_every_row():
    q, k, v, _, idx, kv_lens, sink = _inputs()
    scale = 1 / math.sqrt(16)
    for s_ in (None, sink):
        o_ref, l_ref = sfa_forward(q, k, v, idx, scale, kv_lens=kv_lens, sink=s_, dtype=torch.float64)
        err_o, err_l = fr.compare_fwd(o_ref.float(), l_ref.float(), q, k, v, idx, scale, kv_lens, s_, chunk=7)
        assert err_o < 1e-5 and err_l < 1e-5, (err_o, err_l)


def test_compare_fwd_catches_a_wrong_row():
    q, k, v, _, idx, kv_lens, sink = _inputs(1)
    scale = 0.3
    o_ref, l_ref = sfa_forward(q, k, v, idx, scale, kv_lens=kv_lens, sink=sink)
    bad = o_ref.clone()
    bad[1, 17] = o_ref[1, 16]  # a row written with its neighbour's values
    err_o, _ = fr.compare_fwd(bad, l_ref, q, k, v, idx, scale, kv_lens, sink)
    assert err_o > 0.05


def test_backward_matches_oracle_and_autograd():
    q, k, v, dout, idx, kv_lens, sink = _inputs(2)
    scale = 0.25
    o, l = sfa_forward(q, k, v, idx, scale, kv_lens=kv_lens, sink=sink, dtype=torch.float64)
    ref = sfa_backward(q, k, v, idx, o, l, dout, scale, kv_lens=kv_lens, sink=sink, dtype=torch.float64)
    got = fr.backward(q, k, v, idx, o.float(), l.float(), dout, scale, kv_lens, sink, chunk=6)
    for a, b in zip(got, ref):
        assert float((a.double() - b).abs().max()) < 1e-4
    # a gradient into LSE, against autograd of the oracle's dense restatement
    dlse = torch.randn(l.shape, generator=torch.Generator().manual_seed(7))
    qc, kc, vc = (t.double().requires_grad_(True) for t in (q, k, v))
    sc = sink.double().requires_grad_(True)
    o2, l2 = sfa_forward_autograd(qc, kc, vc, idx, scale=scale, kv_lens=kv_lens, sink=sc)
    ((o2 * dout.double()).sum() + (l2 * dlse.double()).sum()).backward()
    got = fr.backward(q, k, v, idx, o.float(), l.float(), dout, scale, kv_lens, sink, dlse=dlse)
    for a, b in zip(got, (qc.grad, kc.grad, vc.grad, sc.grad)):
        assert float((a.double() - b).abs().max()) < 1e-4


def test_rowwise_error_flags_an_unwritten_row():
    g = torch.Generator().manual_seed(3)
    ref = torch.randn(40, 8, 16, generator=g)
    a = ref + 1e-4 * torch.randn(40, 8, 16, generator=g)
    assert fr.rowwise_rel_err(a, ref) < 1e-3
    a[13, 2] = 0
    assert fr.rowwise_rel_err(a, ref) > 0.99


def test_key_grads_match_the_full_backward():
    """The per-key gradient helper against the full backward's rows (which
    the test above pins to the oracle), for referenced, unreferenced,
    out-of-range and past-kv_lens keys, with a gradient into LSE."""
    q, k, v, dout, idx, kv_lens, sink = _inputs(4)
    scale = 0.3
    o, l = sfa_forward(q, k, v, idx, scale, kv_lens=kv_lens, sink=sink)
    dlse = torch.randn(l.shape, generator=torch.Generator().manual_seed(9))
    _, rk, rv, _ = fr.backward(q, k, v, idx, o, l, dout, scale, kv_lens, sink, dlse=dlse)
    keys = [0, 3, 20, 21, 32, 40]
    for b in range(2):
        for g in range(2):
            dk, dv = fr.key_grads(q, k, v, idx, o, l, dout, scale, keys, b=b, g=g, kv_lens=kv_lens, dlse=dlse,
                                  chunk=3)
            for n, j in enumerate(keys):
                if j < 33:
                    assert float((dk[n] - rk[b, j, g]).abs().max()) < 1e-4, (b, g, j)
                    assert float((dv[n] - rv[b, j, g]).abs().max()) < 1e-4, (b, g, j)
                else:
                    assert bool((dk[n] == 0).all() and (dv[n] == 0).all())
    # a planted mistake (delta without the LSE gradient) is caught
    dk_bad, _ = fr.key_grads(q, k, v, idx, o, l, dout, scale, [3], b=0, g=0, kv_lens=kv_lens)
    assert float((dk_bad[0] - rk[0, 3, 0]).abs().max()) > 1e-3
