"""Full-grid reference for the parity tests: the oracle's math evaluated by
torch in float32 on the tensors' own device.

The CPU oracle (``oracle/sfa_oracle.py``) is the checker; at the full
workload sizes it only finishes on sampled rows.  To check *every* row of a
full-size run (a placement mistake that leaves rows unwritten would escape a
row sample), the tests evaluate the same formulas here, chunked over queries,
on the GPU in float32:

* forward (SFA.py:359-480): ``s = scale·<q, k[idx]>`` over the valid slots
  (``0 <= idx < kv_lens[b]`` or ``Skv``), ``lse = logsumexp(s)`` (joined by the
  sink when given), ``out = Σ exp(s - lse)·v[idx]``; a row without valid slot
  gives ``out = 0``, ``lse = -inf``;
* backward (SFA.py:590-853): ``δ = Σ out·dout - dlse``, ``P = exp(s - lse)``,
  ``dS = P(dP - δ)``, ``dq = scale·Σ dS·k``, ``dk[idx] += scale·dS·q``,
  ``dv[idx] += P·dout`` (``index_add_``), ``dsink = -Σ exp(sink - lse)·δ``.

Every batched product is ``torch.bmm`` on contiguous float32 operands.  This
module is pinned against the CPU oracle on small inputs
(``tests/test_fullgrid_ref.py``), so it is a restatement checked like the
oracle itself, not a second product path.
"""
from __future__ import annotations

import math
from typing import Iterator, Optional, Tuple

import torch


def _bounds(B: int, Skv: int, kv_lens: Optional[torch.Tensor], device) -> torch.Tensor:
    if kv_lens is None:
        return torch.full((B,), Skv, dtype=torch.long, device=device)
    return kv_lens.to(device).long().clamp(max=Skv)


def fwd_chunks(q, k, v, idx, scale, kv_lens=None, sink=None, chunk: int = 64
               ) -> Iterator[Tuple[int, int, int, int, torch.Tensor, torch.Tensor]]:
    """Yields ``(b, s0, s1, g, out, lse)`` per chunk of queries and KV head:
    ``out`` ``[s1 - s0, G, Dv]`` and ``lse`` ``[s1 - s0, G]`` float32 for query
    heads ``g·G .. (g+1)·G - 1``."""
    B, Sq, Hq, Dqk = q.shape
    Skv, Hkv, Dv = k.shape[1], k.shape[2], v.shape[3]
    G = Hq // Hkv
    bound = _bounds(B, Skv, kv_lens, q.device)
    for b in range(B):
        for g in range(Hkv):
            kf = k[b, :, g].float().contiguous()
            vf = v[b, :, g].float().contiguous()
            sk = sink[g * G:(g + 1) * G].float() if sink is not None else None
            for s0 in range(0, Sq, chunk):
                s1 = min(Sq, s0 + chunk)
                ib = idx[b, s0:s1, g].long()
                vm = (ib >= 0) & (ib < bound[b])
                safe = torch.where(vm, ib, torch.zeros_like(ib))
                kg = kf[safe]                                        # [C, K, Dqk]
                vg = vf[safe]                                        # [C, K, Dv]
                qg = q[b, s0:s1, g * G:(g + 1) * G].float().contiguous()
                s = torch.bmm(qg, kg.transpose(1, 2).contiguous()) * scale   # [C, G, K]
                s = s.masked_fill(~vm[:, None, :], -math.inf)
                lse = torch.logsumexp(s, dim=-1)
                if sk is not None:
                    lse = torch.logaddexp(lse, sk[None, :].expand_as(lse))
                lfin = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
                p = torch.exp(s - lfin[..., None])
                p = torch.where(vm[:, None, :], p, torch.zeros_like(p))
                yield b, s0, s1, g, torch.bmm(p, vg), lse


def compare_fwd(out, lse, q, k, v, idx, scale, kv_lens=None, sink=None, chunk: int = 64) -> Tuple[float, float]:
    """Max-abs error of ``out`` and of the finite ``lse`` entries over every
    row against the float32 evaluation; raises AssertionError when the two
    disagree on which LSE entries are finite (or ``out`` holds a NaN)."""
    G = q.shape[2] // k.shape[2]
    err_o, err_l = 0.0, 0.0
    for b, s0, s1, g, o_ref, l_ref in fwd_chunks(q, k, v, idx, scale, kv_lens, sink, chunk):
        o = out[b, s0:s1, g * G:(g + 1) * G].float()
        l = lse[b, s0:s1, g * G:(g + 1) * G].float()
        fin = torch.isfinite(l_ref)
        if not torch.equal(torch.isfinite(l), fin):
            raise AssertionError(f"LSE finiteness differs in rows {s0}..{s1} of batch {b}, kv head {g}")
        if bool(torch.isnan(o).any()):
            raise AssertionError(f"NaN in out rows {s0}..{s1} of batch {b}, kv head {g}")
        err_o = max(err_o, float((o - o_ref).abs().max()))
        if bool(fin.any()):
            err_l = max(err_l, float((l[fin] - l_ref[fin]).abs().max()))
    return err_o, err_l


def backward(q, k, v, idx, out, lse, dout, scale, kv_lens=None, sink=None, dlse=None, chunk: int = 256):
    """``(dq, dk, dv, dsink)`` float32 on the inputs' device (``dsink`` None
    without a sink); ``out`` / ``lse`` are the forward's results."""
    B, Sq, Hq, Dqk = q.shape
    Skv, Hkv, Dv = k.shape[1], k.shape[2], v.shape[3]
    G = Hq // Hkv
    dev = q.device
    bound = _bounds(B, Skv, kv_lens, dev)
    dq = torch.zeros(B, Sq, Hq, Dqk, dtype=torch.float32, device=dev)
    dk = torch.zeros(B, Skv, Hkv, Dqk, dtype=torch.float32, device=dev)
    dv = torch.zeros(B, Skv, Hkv, Dv, dtype=torch.float32, device=dev)
    dsink = torch.zeros(Hq, dtype=torch.float32, device=dev) if sink is not None else None
    for b in range(B):
        for g in range(Hkv):
            kf = k[b, :, g].float().contiguous()
            vf = v[b, :, g].float().contiguous()
            hs = slice(g * G, (g + 1) * G)
            for s0 in range(0, Sq, chunk):
                s1 = min(Sq, s0 + chunk)
                ib = idx[b, s0:s1, g].long()
                vm = (ib >= 0) & (ib < bound[b])
                safe = torch.where(vm, ib, torch.zeros_like(ib))
                kg = kf[safe]
                vg = vf[safe]
                qg = q[b, s0:s1, hs].float().contiguous()
                og = out[b, s0:s1, hs].float()
                dog = dout[b, s0:s1, hs].float().contiguous()
                lg = lse[b, s0:s1, hs].float()
                lfin = torch.where(torch.isfinite(lg), lg, torch.zeros_like(lg))
                delta = (og * dog).sum(-1)
                if dlse is not None:
                    delta = delta - dlse[b, s0:s1, hs].float()
                s = torch.bmm(qg, kg.transpose(1, 2).contiguous()) * scale
                p = torch.exp(s - lfin[..., None])
                p = torch.where(vm[:, None, :] & torch.isfinite(lg)[..., None], p, torch.zeros_like(p))
                dp = torch.bmm(dog, vg.transpose(1, 2).contiguous())
                ds = p * (dp - delta[..., None])
                dq[b, s0:s1, hs] = scale * torch.bmm(ds, kg)
                dk_c = scale * torch.bmm(ds.transpose(1, 2).contiguous(), qg)      # [C, K, Dqk]
                dv_c = torch.bmm(p.transpose(1, 2).contiguous(), dog)            # [C, K, Dv]
                w = vm.reshape(-1)
                rows = safe.reshape(-1)[w]
                dk[b, :, g].index_add_(0, rows, dk_c.reshape(-1, Dqk)[w])
                dv[b, :, g].index_add_(0, rows, dv_c.reshape(-1, Dv)[w])
                if sink is not None:
                    sg = sink[hs].float()
                    ps = torch.where(torch.isfinite(lg), torch.exp(sg[None, :] - lfin), torch.zeros_like(lg))
                    dsink[hs] -= (ps * delta).sum(0)
    return dq, dk, dv, dsink


def rowwise_rel_err(a: torch.Tensor, ref: torch.Tensor, floor: float = 1e-3) -> float:
    """Largest per-row relative L2 error over the rows (last dim) whose
    reference norm exceeds ``floor`` times the median row norm; a row left
    unwritten (or written with another row's values) gives an error near 1."""
    a = a.float().reshape(-1, a.shape[-1])
    ref = ref.float().reshape(-1, ref.shape[-1])
    rn = ref.norm(dim=1)
    keep = rn > floor * rn.median().clamp_min(1e-30)
    err = (a - ref).norm(dim=1)[keep] / rn[keep]
    return float(err.max()) if err.numel() else 0.0


def key_grads(q, k, v, idx, out, lse, dout, scale, keys, b: int = 0, g: int = 0, kv_lens=None, dlse=None,
              chunk: int = 512):
    """``(dk, dv)`` float32 ``[len(keys), Dqk]`` / ``[len(keys), Dv]``: the
    gradients of key rows ``keys`` of batch ``b``, KV head ``g``, summed over
    every (query, slot) pair that references them (SFA.py:831-853), each pair
    with its own query's P and dS from ``lse`` and ``delta = Σ out·dout -
    dlse``.  This checks a key's gradient at full workload sizes without the
    whole backward: only the queries that select the key are visited."""
    Sq, Hq, Dqk = q.shape[1], q.shape[2], q.shape[3]
    Skv, Hkv, Dv = k.shape[1], k.shape[2], v.shape[3]
    G = Hq // Hkv
    dev = q.device
    hs = slice(g * G, (g + 1) * G)
    bound = int(_bounds(q.shape[0], Skv, kv_lens, dev)[b])
    ib = idx[b, :, g].long()
    vm = (ib >= 0) & (ib < bound)
    dk = torch.zeros(len(keys), Dqk, dtype=torch.float32, device=dev)
    dv = torch.zeros(len(keys), Dv, dtype=torch.float32, device=dev)
    for n, j in enumerate(keys):
        j = int(j)
        if not 0 <= j < bound:
            continue
        ts = ((ib == j) & vm).nonzero(as_tuple=True)[0]  # one entry per referencing slot
        kj = k[b, j, g].float()
        vj = v[b, j, g].float()
        for c0 in range(0, ts.numel(), chunk):
            t = ts[c0:c0 + chunk]
            qg = q[b, t][:, hs].float()                           # [n, G, Dqk]
            dog = dout[b, t][:, hs].float()                       # [n, G, Dv]
            lg = lse[b, t][:, hs].float()
            delta = (out[b, t][:, hs].float() * dog).sum(-1)
            if dlse is not None:
                delta = delta - dlse[b, t][:, hs].float()
            lfin = torch.where(torch.isfinite(lg), lg, torch.zeros_like(lg))
            p = torch.exp(qg @ kj * scale - lfin)
            p = torch.where(torch.isfinite(lg), p, torch.zeros_like(p))
            ds = p * (dog @ vj - delta)
            dk[n] += scale * (ds[..., None] * qg).sum((0, 1))
            dv[n] += (p[..., None] * dog).sum((0, 1))
    return dk, dv
