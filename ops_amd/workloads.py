"""Seeded synthetic inputs for the sparse-attention workloads.

The reference (SFA.py) is driven by a model layer that produces per-query
top-k KV row ids (its docstring, SFA.py:86-94); none is shipped.  This module
plays that caller for five workloads:

``tiny``         B=1, S=256, Hq=4, Hkv=1, d=64, top-k 64, fp32, fwd+bwd
``prefill``      B=1, S=4096, Hq=16, Hkv=1 (MQA), d=128, top-k 512, bf16
``train_gqa``    B=2, S=8192, Hq=32, Hkv=2, d=128, top-k 1024, bf16, fwd+bwd,
                 10 % of key positions receive ≈40 % of references
``mla_prefill``  B=1, S=32768, Hq=128, one latent KV head, d_qk=576, d_v=512
                 (V = first 512 dims of K), top-k 2048, bf16
``mla_decode``   B=64, 1 query each, Hq=128, KV cache [64, 65536, 1, 576],
                 context lengths U{16384..65536}, top-k 2048, bf16

Index rows are int32 with ``-1`` padding after the valid slots; valid slots are
in random order (sampling without replacement uses random-key top-k; weighted
sampling uses Efraimidis–Spirakis keys ``log(u)/w``).  Every tensor comes from
its own ``torch.Generator`` seeded from (seed, tensor id), so a workload is
reproducible on any device at any chunking.  ``shrink`` variants keep each
workload's structure at sizes the CPU oracle finishes in seconds.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, Optional

import torch

__all__ = ["Workload", "make_workload", "WORKLOADS", "workload_spec"]


@dataclass
class Workload:
    name: str
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    idx: torch.Tensor
    scale: float
    kv_lens: Optional[torch.Tensor] = None
    dout: Optional[torch.Tensor] = None
    meta: Dict = field(default_factory=dict)

    @property
    def G(self) -> int:
        return self.q.shape[2] // self.k.shape[2]


# name -> full-size parameters
WORKLOADS = {
    "tiny": dict(B=1, S=256, Hq=4, Hkv=1, Dqk=64, Dv=64, K=64, dtype=torch.float32, bwd=True),
    "prefill": dict(B=1, S=4096, Hq=16, Hkv=1, Dqk=128, Dv=128, K=512, dtype=torch.bfloat16, bwd=False),
    "train_gqa": dict(B=2, S=8192, Hq=32, Hkv=2, Dqk=128, Dv=128, K=1024, dtype=torch.bfloat16, bwd=True),
    "mla_prefill": dict(B=1, S=32768, Hq=128, Hkv=1, Dqk=576, Dv=512, K=2048, dtype=torch.bfloat16, bwd=False),
    "mla_decode": dict(B=64, S=1, Skv=65536, Hq=128, Hkv=1, Dqk=576, Dv=512, K=2048,
                       ctx_lo=16384, dtype=torch.bfloat16, bwd=False),
}


def workload_spec(name: str, **overrides) -> dict:
    spec = dict(WORKLOADS[name])
    spec.update(overrides)
    return spec


def _gen(device, seed: int, tid: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed * 1_000_003 + tid)
    return g


def _context_lens(spec: dict, Skv: int, device, seed: int) -> torch.Tensor:
    """Decode context lengths: uniform in [ctx_lo, Skv] per sequence (int64)."""
    lo = spec.get("ctx_lo", Skv // 4)
    return torch.randint(lo, Skv + 1, (spec["B"],), generator=_gen(device, seed, 5), device=device,
                         dtype=torch.int64)


def decode_context_lens(device="cpu", seed: int = 0, **overrides) -> torch.Tensor:
    """The mla_decode workload's kv_lens (int32 ``[B]``) without building its
    cache: the same draw as ``make_workload("mla_decode", ...).kv_lens``."""
    spec = workload_spec("mla_decode", **overrides)
    return _context_lens(spec, spec["Skv"], device, seed).to(torch.int32)


def _randn(shape, dtype, device, gen, chunk_rows: int = 1 << 22):
    """N(0,1) drawn in fp32 then cast, in chunks along dim 0's flattened rows."""
    out = torch.empty(shape, dtype=dtype, device=device)
    flat = out.view(-1, shape[-1])
    for r0 in range(0, flat.shape[0], max(1, chunk_rows // shape[-1])):
        r1 = min(flat.shape[0], r0 + max(1, chunk_rows // shape[-1]))
        flat[r0:r1] = torch.randn((r1 - r0, shape[-1]), generator=gen, device=device,
                                  dtype=torch.float32).to(dtype)
    return out


def _topk_keys(keys: torch.Tensor, m: int) -> torch.Tensor:
    """Positions of the m largest keys per row (random order w.r.t. position)."""
    return torch.topk(keys, m, dim=-1, sorted=True).indices


def _rows_chunk(n_rows: int, row_len: int, budget: int = 1 << 24) -> int:
    return max(1, min(n_rows, budget // max(row_len, 1)))


def _causal_uniform(S: int, K: int, device, gen) -> torch.Tensor:
    """Row t: min(K, t+1) positions drawn uniformly without replacement from
    [0, t]; -1 after them."""
    idx = torch.full((S, K), -1, dtype=torch.int32, device=device)
    C = _rows_chunk(S, S)
    pos = torch.arange(S, device=device)
    for t0 in range(0, S, C):
        t1 = min(S, t0 + C)
        t = torch.arange(t0, t1, device=device)
        u = torch.rand((t1 - t0, S), generator=gen, device=device)
        allowed = pos[None, :] <= t[:, None]
        u = torch.where(allowed, u, torch.full_like(u, -1.0))
        kk = min(K, S)
        sel = _topk_keys(u, kk).to(torch.int32)
        nvalid = torch.clamp(t + 1, max=K)
        slot = torch.arange(kk, device=device)
        sel = torch.where(slot[None, :] < nvalid[:, None], sel, torch.full_like(sel, -1))
        idx[t0:t1, :kk] = sel
    return idx


def _prefill_window(S: int, K: int, window: int, device, gen) -> torch.Tensor:
    """Row t: {max(0, t-window+1) .. t} plus min(K-window, max(0, t-window+1))
    uniform draws without replacement from [0, t-window]; -1 after them."""
    idx = torch.full((S, K), -1, dtype=torch.int32, device=device)
    C = _rows_chunk(S, S)
    pos = torch.arange(S, device=device)
    nrand_max = K - window
    for t0 in range(0, S, C):
        t1 = min(S, t0 + C)
        t = torch.arange(t0, t1, device=device)
        # window part, newest first
        w = t[:, None] - torch.arange(window, device=device)[None, :]
        wvalid = w >= 0
        # random part from [0, t-window]
        u = torch.rand((t1 - t0, S), generator=gen, device=device)
        allowed = pos[None, :] <= (t[:, None] - window)
        u = torch.where(allowed, u, torch.full_like(u, -1.0))
        kr = min(nrand_max, S)
        sel = _topk_keys(u, kr)
        nrand = torch.clamp(t - window + 1, min=0, max=nrand_max)
        rvalid = torch.arange(kr, device=device)[None, :] < nrand[:, None]
        cand = torch.cat([w, sel], dim=1)
        cvalid = torch.cat([wvalid, rvalid], dim=1)
        # shuffle valid entries to random slot order, then compact valid first
        perm_keys = torch.rand(cand.shape, generator=gen, device=device)
        perm_keys = torch.where(cvalid, perm_keys, torch.full_like(perm_keys, -1.0))
        order = torch.sort(perm_keys, dim=1, descending=True).indices
        cand = torch.gather(cand, 1, order)
        cvalid = torch.gather(cvalid, 1, order)
        cand = torch.where(cvalid, cand, torch.full_like(cand, -1))
        idx[t0:t1] = cand[:, :K].to(torch.int32)
    return idx


def _weighted_causal(S: int, K: int, hot: torch.Tensor, w_hot: float, device, gen,
                     rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Row t: min(K, t+1) draws without replacement from [0, t] with weight
    w_hot on hot positions and 1 elsewhere (Efraimidis–Spirakis keys)."""
    rows = torch.arange(S, device=device) if rows is None else rows
    n = rows.numel()
    idx = torch.full((n, K), -1, dtype=torch.int32, device=device)
    C = _rows_chunk(n, S)
    pos = torch.arange(S, device=device)
    logw = torch.where(hot, torch.full((S,), math.log(w_hot), device=device),
                       torch.zeros((S,), device=device))
    for r0 in range(0, n, C):
        r1 = min(n, r0 + C)
        t = rows[r0:r1]
        u = torch.rand((r1 - r0, S), generator=gen, device=device, dtype=torch.float64)
        keys = torch.log(u.clamp_min(1e-300)) * torch.exp(-logw.double())[None, :]
        allowed = pos[None, :] <= t[:, None]
        keys = torch.where(allowed, keys, torch.full_like(keys, -math.inf))
        kk = min(K, S)
        sel = _topk_keys(keys, kk).to(torch.int32)
        nvalid = torch.clamp(t + 1, max=K)
        sel = torch.where(torch.arange(kk, device=device)[None, :] < nvalid[:, None], sel,
                          torch.full_like(sel, -1))
        idx[r0:r1, :kk] = sel
    return idx


def _hot_share(idx: torch.Tensor, hot: torch.Tensor) -> float:
    v = idx >= 0
    h = hot[idx.clamp_min(0).long()] & v
    return float(h.sum().item()) / max(1, int(v.sum().item()))


def _calibrate_w_hot(S, K, hot, device, seed, target=0.40, sample_stride=None):
    """Bisection on log(w_hot) so hot positions receive ``target`` of the
    references (measured on a strided sample of query rows)."""
    stride = sample_stride or max(1, S // 256)
    rows = torch.arange(0, S, stride, device=device)
    lo, hi = 0.0, math.log(1e6)
    for it in range(24):
        mid = 0.5 * (lo + hi)
        gen = _gen(device, seed, 9000 + it)
        share = _hot_share(_weighted_causal(S, K, hot, math.exp(mid), device, gen, rows), hot)
        if share < target:
            lo = mid
        else:
            hi = mid
    return math.exp(0.5 * (lo + hi))


def _mla_prefill_idx(S: int, K: int, recent_win: int, n_recent: int, device, gen) -> torch.Tensor:
    """Row t: if t+1 <= K all of [0, t] (random order) then -1; otherwise
    n_recent uniform from [t-recent_win+1, t] plus K-n_recent uniform from the
    rest of [0, t]."""
    idx = torch.full((S, K), -1, dtype=torch.int32, device=device)
    C = _rows_chunk(S, S)
    pos = torch.arange(S, device=device)
    for t0 in range(0, S, C):
        t1 = min(S, t0 + C)
        t = torch.arange(t0, t1, device=device)
        u = torch.rand((t1 - t0, S), generator=gen, device=device)
        causal = pos[None, :] <= t[:, None]
        recent = causal & (pos[None, :] > t[:, None] - recent_win)
        short = (t + 1) <= K
        # recent draws: n_recent from the window (long rows only)
        ur = torch.where(recent, u, torch.full_like(u, -1.0))
        sel_r = _topk_keys(ur, min(n_recent, S))
        # mark the chosen recent ones as not allowed for the rest
        taken = torch.zeros_like(causal)
        taken.scatter_(1, sel_r, True)
        taken &= recent
        u2 = torch.rand((t1 - t0, S), generator=gen, device=device)
        rest_allowed = causal & ~taken
        rest_allowed = torch.where(short[:, None], causal, rest_allowed)
        u2 = torch.where(rest_allowed, u2, torch.full_like(u2, -1.0))
        sel_rest = _topk_keys(u2, min(K, S))  # long rows use the first K-n_recent
        kk = min(K, S)
        slot = torch.arange(kk, device=device)[None, :]
        long_row = torch.cat([sel_r, sel_rest[:, :kk - n_recent]], dim=1) if kk > n_recent else sel_r[:, :kk]
        nvalid = torch.clamp(t + 1, max=K)
        short_row = torch.where(slot < nvalid[:, None], sel_rest, torch.full_like(sel_rest, -1))
        row = torch.where(short[:, None], short_row, long_row)
        # shuffle slot order of long rows so recent and uniform draws interleave
        pk = torch.rand(row.shape, generator=gen, device=device)
        pk = torch.where(row >= 0, pk, torch.full_like(pk, -1.0))
        order = torch.sort(pk, dim=1, descending=True).indices
        idx[t0:t1, :kk] = torch.gather(row, 1, order).to(torch.int32)
    return idx


def _decode_idx(B: int, K: int, ctx: torch.Tensor, Skv: int, device, gen) -> torch.Tensor:
    """Per sequence: K positions uniform without replacement from [0, ctx[b])."""
    idx = torch.full((B, K), -1, dtype=torch.int32, device=device)
    pos = torch.arange(Skv, device=device)
    C = _rows_chunk(B, Skv)
    for b0 in range(0, B, C):
        b1 = min(B, b0 + C)
        u = torch.rand((b1 - b0, Skv), generator=gen, device=device)
        u = torch.where(pos[None, :] < ctx[b0:b1, None], u, torch.full_like(u, -1.0))
        kk = min(K, Skv)
        sel = _topk_keys(u, kk).to(torch.int32)
        valid = torch.arange(kk, device=device)[None, :] < ctx[b0:b1, None]
        idx[b0:b1, :kk] = torch.where(valid, sel, torch.full_like(sel, -1))
    return idx


def make_workload(name: str, device="cpu", seed: int = 0, with_dout: Optional[bool] = None,
                  dtype: Optional[torch.dtype] = None, **overrides) -> Workload:
    """Build workload ``name`` (see module docstring) on ``device``.

    ``overrides`` shrink the shapes (S, K, Hq, Hkv, Dqk, Dv, B, Skv, ...);
    the index recipe keeps its structure (windows and recency widths scale
    with K).
    """
    spec = workload_spec(name, **overrides)
    dt = dtype or spec["dtype"]
    B, Hq, Hkv, Dqk, Dv, K = spec["B"], spec["Hq"], spec["Hkv"], spec["Dqk"], spec["Dv"], spec["K"]
    S = spec["S"]
    bwd = spec["bwd"] if with_dout is None else with_dout
    meta = {"spec": {k: (str(v) if isinstance(v, torch.dtype) else v) for k, v in spec.items()}}
    kv_lens = None

    if name in ("mla_prefill", "mla_decode"):
        Skv = spec.get("Skv", S)
        q = _randn((B, S, Hq, Dqk), dt, device, _gen(device, seed, 1))
        kv = _randn((B, Skv, Hkv, Dqk), dt, device, _gen(device, seed, 2))
        k, v = kv, kv[..., :Dv]
        scale = 1.0 / math.sqrt(Dqk)
        if name == "mla_prefill":
            n_recent = spec.get("n_recent", K // 8)
            win = spec.get("recent_win", K // 2)
            gidx = _mla_prefill_idx(S, K, win, n_recent, device, _gen(device, seed, 4))
            idx = gidx.view(1, S, 1, K).expand(B, S, Hkv, K).contiguous()
        else:
            ctx = _context_lens(spec, Skv, device, seed)
            kv_lens = ctx.to(torch.int32)
            gidx = _decode_idx(B, K, ctx, Skv, device, _gen(device, seed, 4))
            idx = gidx.view(B, 1, 1, K).expand(B, 1, Hkv, K).contiguous()
            meta["ctx_lens"] = ctx.tolist()
    else:
        q = _randn((B, S, Hq, Dqk), dt, device, _gen(device, seed, 1))
        k = _randn((B, S, Hkv, Dqk), dt, device, _gen(device, seed, 2))
        v = _randn((B, S, Hkv, Dv), dt, device, _gen(device, seed, 3))
        scale = 1.0 / math.sqrt(Dqk)
        if name == "tiny":
            idx = torch.stack([
                torch.stack([_causal_uniform(S, K, device, _gen(device, seed, 100 + b * 64 + g))
                             for g in range(Hkv)], dim=1)
                for b in range(B)])
        elif name == "prefill":
            window = spec.get("window", K // 8)
            idx = torch.stack([
                torch.stack([_prefill_window(S, K, window, device, _gen(device, seed, 100 + b * 64 + g))
                             for g in range(Hkv)], dim=1)
                for b in range(B)])
        elif name == "train_gqa":
            hot_frac = spec.get("hot_frac", 0.10)
            target = spec.get("hot_share", 0.40)
            rows_b = []
            shares, whots = [], []
            for b in range(B):
                rows_g = []
                for g in range(Hkv):
                    gh = _gen(device, seed, 200 + b * 64 + g)
                    n_hot = max(1, int(round(hot_frac * S)))
                    hot = torch.zeros(S, dtype=torch.bool, device=device)
                    hot[torch.randperm(S, generator=gh, device=device)[:n_hot]] = True
                    w_hot = _calibrate_w_hot(S, K, hot, device, seed * 131 + b * 64 + g, target)
                    ig = _weighted_causal(S, K, hot, w_hot, device, _gen(device, seed, 100 + b * 64 + g))
                    shares.append(_hot_share(ig, hot))
                    whots.append(w_hot)
                    rows_g.append(ig)
                rows_b.append(torch.stack(rows_g, dim=1))
            idx = torch.stack(rows_b)
            meta["hot_share"] = shares
            meta["w_hot"] = whots
        else:
            raise KeyError(name)
    dout = _randn(tuple(q.shape[:3]) + (Dv,), dt, device, _gen(device, seed, 6)) if bwd else None
    return Workload(name=name, q=q, k=k, v=v, idx=idx.contiguous(), scale=scale, kv_lens=kv_lens,
                    dout=dout, meta=meta)


def page_kv(k: torch.Tensor, v: torch.Tensor, page_size: int, seed: int = 0, spare_pages: int = 0):
    """Paged copy of a contiguous cache for the paged-KV forward.

    ``k`` ``[B, Skv, Hkv, Dqk]`` / ``v`` ``[B, Skv, Hkv, Dv]`` (``v`` may be a
    prefix view of ``k``, as in MLA) are cut into pages of ``page_size`` rows
    that are scattered over a pool in a seeded random order, with
    ``spare_pages`` extra pages of noise.  Returns ``(k_pool, v_pool,
    block_table)``: pools ``[num_pages, page_size, Hkv, D]`` (``v_pool`` a
    prefix view of ``k_pool`` when ``v`` is one of ``k``) and the
    ``[B, Skv / page_size]`` int32 block table that maps them back.
    """
    B, Skv, Hkv, Dqk = k.shape
    if Skv % page_size:
        raise ValueError("Skv must be a multiple of page_size")
    npb = Skv // page_size
    n = B * npb + spare_pages
    g = _gen(k.device, seed, 7)
    perm = torch.randperm(n, generator=g, device=k.device)       # pool slot -> logical page (>= B*npb: spare)
    where = torch.empty_like(perm)
    where[perm] = torch.arange(n, device=k.device)               # logical page -> pool slot
    block_table = where[:B * npb].view(B, npb).to(torch.int32).contiguous()

    def pool_of(x):
        pages = x.reshape(B * npb, page_size, Hkv, x.shape[3])
        if spare_pages:
            noise = _randn((spare_pages, page_size, Hkv, x.shape[3]), x.dtype, x.device, _gen(x.device, seed, 8))
            pages = torch.cat([pages, noise])
        return pages[perm].contiguous()

    shares_storage = v.data_ptr() == k.data_ptr() and v.stride() == k.stride()
    k_pool = pool_of(k)
    v_pool = k_pool[..., :v.shape[3]] if shares_storage else pool_of(v)
    return k_pool, v_pool, block_table

