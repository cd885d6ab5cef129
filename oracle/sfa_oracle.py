"""CPU restatement of top-k sparse flash attention (SFA) — test infrastructure only.

This module is the reference the HIP kernels in ``ops_amd`` are compared
against: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it, and never as the thing measured or shipped.  The product path
(``ops_amd.sfa``) never calls into it.

It restates, in plain PyTorch eager on the CPU, the math of the reference
``SFA.py`` (lilac-me/ops):

* forward  — ``_inner_fwd`` SFA.py:359-480 (gather top-k rows, masked base-2
  online softmax, P·V, attention sink, LSE) driven by ``_attn_fwd`` SFA.py:483-587;
* delta    — ``_get_delta_split`` SFA.py:590-610 (δ = Σ_d O·dO);
* dQ       — ``_inner_dq`` SFA.py:613-716 (P = 2^(s·c − lse2), dS = P(dP − δ),
  dQ = scale·dS·K);
* dK/dV    — ``_inner_dkv`` SFA.py:719-853 (dV += Pᵀ·dO, dK += scale·dSᵀ·Q,
  scattered with ``atomic_add`` into the referenced rows, SFA.py:851-853);
* dsink    — SFA.py:964-970 (dsink = −Σ 2^(sink·log2e − lse2)·δ).

Generalisations relative to the reference (the drop-in boundary's API):

* BSHD layout with separate ``k`` and ``v`` (the reference has one ``kv`` tensor
  that is both, SFA.py:116, 425, 456) and ``Hkv`` KV heads with per-(b, kv-head,
  query) index rows; query head ``h`` reads KV head ``h // (Hq // Hkv)``.
* Validity of a slot is ``0 <= idx < bound`` where ``bound`` is ``kv_lens[b]`` if
  given, else ``Skv``.  The reference tests ``idx >= 0`` and ``slot < TOPK_eff``
  (SFA.py:394-396, 403-404) with no upper bound; ``TOPK_eff`` (SFA.py:62-66) only
  drops slots after the largest valid count, which never happens with trailing
  ``-1`` padding, so for every index row the reference can address the two rules
  select the same slots.
* LSE is returned in natural-log units (the reference keeps ``lse2 = m + log2 l``
  in base 2, SFA.py:474; ``lse = lse2 · ln 2``).  A row with no valid slot gives
  ``O = 0`` and ``LSE = -inf`` (the reference's sentinel is ≈ −1e11, SFA.py:381).
* The attention sink is optional (``sink=None`` ≡ sink = −∞).
* Paged KV caches (``paged_to_contiguous``): not in the reference, whose
  ``_attn_fwd`` reads one contiguous kv tensor (SFA.py:483-587).  The serving
  layout is restated as a plain mapping back to the contiguous cache: logical
  key ``i`` of sequence ``b`` is row ``i % page_size`` of pool page
  ``block_table[b, i // page_size]``; a slot whose page id lies outside
  ``[0, num_pages)`` is invalid.  The forward over a paged cache is then
  ``sfa_forward`` of the mapped cache and indices.
* Top-k index producer (``indexer_scores``, ``indexer_topk``): also not in the
  reference, which consumes its result (``topk_idxs``, SFA.py:88-90).  The
  scores restate DeepSeek-V3.2's lightning indexer,
  ``I[b,t,s] = sum_h w[b,t,h] * relu(<q[b,t,h], k[b,s]>)`` over the keys
  ``s <= t + L_b - Sq``; a row keeps its ``topk`` best keys (equal scores: the
  lower key first) in ascending key order, then ``-1``.

Duplicated indices are counted once per slot, as in the reference, which
processes every slot independently (SFA.py:386-467).

Every function computes in ``dtype`` (float32 by default; float64 for pinning
the float32 path).  Work is chunked over queries so that the gathered rows of a
chunk stay within ``max_chunk_bytes``.

Pinning (tests/test_oracle.py): a pure-Python fp64 loop brute force on tiny
inputs, ``torch.nn.functional.scaled_dot_product_attention`` on the dense causal
special case, ``torch.autograd.gradcheck`` of an autograd restatement in fp64,
the explicit backward against autograd, closed forms (single index, q = 0,
duplicates, sink), exact index invariants, and the golden fixtures under
``tests/golden``.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

LOG2E = 1.4426950408889634  # SFA.py:13
LN2 = 0.6931471805599453

__all__ = [
    "sfa_forward",
    "sfa_backward",
    "sfa_forward_autograd",
    "valid_mask",
    "count_valid_pairs",
    "paged_to_contiguous",
    "indexer_key_end",
    "indexer_scores",
    "indexer_topk",
]


def _check_shapes(q, k, v, idx):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or idx.dim() != 4:
        raise ValueError("q, k, v, idx must be 4-D (BSHD; idx is [B, Sq, Hkv, K])")
    B, Sq, Hq, Dqk = q.shape
    Bk, Skv, Hkv, Dk = k.shape
    Bv, Skv2, Hkv2, Dv = v.shape
    if (Bk, Dk) != (B, Dqk) or (Bv, Skv2, Hkv2) != (Bk, Skv, Hkv):
        raise ValueError("shape mismatch between q, k, v")
    if idx.shape[:3] != (B, Sq, Hkv):
        raise ValueError("idx must be [B, Sq, Hkv, K]")
    if Hq % Hkv != 0:
        raise ValueError("Hq must be a multiple of Hkv")
    return B, Sq, Hq, Dqk, Skv, Hkv, Dv, idx.shape[3]


def valid_mask(idx: torch.Tensor, Skv: int, kv_lens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Slot validity ``0 <= idx < bound`` (SFA.py:394-396 plus the upper bound)."""
    idx = idx.long()
    if kv_lens is None:
        bound = torch.full((idx.shape[0],), Skv, dtype=torch.long, device=idx.device)
    else:
        bound = kv_lens.long().clamp(max=Skv).to(idx.device)
    bound = bound.view(-1, *([1] * (idx.dim() - 1)))
    return (idx >= 0) & (idx < bound)


def count_valid_pairs(idx: torch.Tensor, Skv: int, kv_lens: Optional[torch.Tensor] = None) -> int:
    """Number of valid (b, kv-head, query, slot) pairs — the FLOP-counting basis."""
    return int(valid_mask(idx, Skv, kv_lens).sum().item())


def _gather_rows(rows: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """``rows[ids]`` for a 2-D ``rows`` (one index_select over the flattened
    ids: the same values as advanced indexing, many times faster on the CPU)."""
    return rows.index_select(0, ids.reshape(-1)).view(*ids.shape, rows.shape[-1])


def _chunk_size(Sq, G, K, D, esize, max_chunk_bytes):
    per_q = K * D * esize * 3 + G * K * esize * 4
    return max(1, min(Sq, max_chunk_bytes // max(per_q, 1)))


def sfa_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    idx: torch.Tensor,
    scale: Optional[float] = None,
    kv_lens: Optional[torch.Tensor] = None,
    sink: Optional[torch.Tensor] = None,
    dtype: torch.dtype = torch.float32,
    max_chunk_bytes: int = 1 << 28,
    query_chunks: Optional[list] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Forward: returns ``(out [B,Sq,Hq,Dv], lse [B,Sq,Hq])`` in ``dtype``.

    Follows ``_inner_fwd`` SFA.py:359-480 with the exact (non-online) softmax,
    which the online recurrence SFA.py:438-467 evaluates: with ``s = scale·⟨q,k⟩``
    on valid slots, ``lse = log Σ exp(s) (+ exp(sink))`` and
    ``out = Σ exp(s − lse)·v``.  ``query_chunks`` (list of (b, start, stop))
    restricts the work to those query ranges (used to time a bounded sample);
    rows outside them are left at zero.
    """
    B, Sq, Hq, Dqk, Skv, Hkv, Dv, K = _check_shapes(q, k, v, idx)
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(Dqk)  # SFA.py:181-182 default, applied to forward as well
    out = torch.zeros(B, Sq, Hq, Dv, dtype=dtype)
    lse = torch.full((B, Sq, Hq), -math.inf, dtype=dtype)
    valid = valid_mask(idx, Skv, kv_lens)
    C = _chunk_size(Sq, G, K, max(Dqk, Dv), torch.finfo(dtype).bits // 8, max_chunk_bytes)
    ranges = query_chunks
    if ranges is None:
        ranges = [(b, s0, min(Sq, s0 + C)) for b in range(B) for s0 in range(0, Sq, C)]
    for (b, s0, s1) in ranges:
        for g in range(Hkv):
            kb = k[b, :, g].to(dtype)
            vb = v[b, :, g].to(dtype)
            vm = valid[b, s0:s1, g]                                  # [C, K]
            safe = torch.where(vm, idx[b, s0:s1, g].long(), torch.zeros_like(vm, dtype=torch.long))
            kg = _gather_rows(kb, safe)                             # [C, K, Dqk]  gather, SFA.py:407-415
            vg = _gather_rows(vb, safe)                             # [C, K, Dv]
            qg = q[b, s0:s1, g * G:(g + 1) * G].to(dtype)          # [C, G, Dqk]
            s = torch.einsum("cgd,ckd->cgk", qg, kg) * scale        # SFA.py:425, 435
            s = s.masked_fill(~vm[:, None, :], -math.inf)          # SFA.py:436 (−1e11 there)
            l = torch.logsumexp(s, dim=-1)                          # [C, G]
            if sink is not None:                                    # SFA.py:469-474
                l = torch.logaddexp(l, sink[g * G:(g + 1) * G].to(dtype)[None, :])
            lfin = torch.where(torch.isfinite(l), l, torch.zeros_like(l))
            p = torch.exp(s - lfin[..., None])
            p = torch.where(vm[:, None, :], p, torch.zeros_like(p))
            o = torch.einsum("cgk,ckd->cgd", p, vg)                 # SFA.py:456, 478
            out[b, s0:s1, g * G:(g + 1) * G] = o
            lse[b, s0:s1, g * G:(g + 1) * G] = l
    return out, lse


def sfa_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    idx: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    dout: torch.Tensor,
    scale: Optional[float] = None,
    kv_lens: Optional[torch.Tensor] = None,
    sink: Optional[torch.Tensor] = None,
    dtype: torch.dtype = torch.float32,
    max_chunk_bytes: int = 1 << 28,
):
    """Explicit backward: returns ``(dq, dk, dv, dsink)`` in ``dtype``.

    δ = Σ_d O·dO (SFA.py:590-610); P = exp(s − lse) (SFA.py:688-689 in base 2);
    dP = dO·vᵀ; dS = P·(dP − δ) (SFA.py:697); dQ = scale·Σ dS·k (SFA.py:708-714);
    dV[i] += P·dO and dK[i] += scale·dS·q summed over every (query, head, slot)
    that references row i (SFA.py:831-853); dsink = −Σ exp(sink − lse)·δ
    (SFA.py:964-970).  ``dsink`` is ``None`` when ``sink`` is ``None``.
    """
    B, Sq, Hq, Dqk, Skv, Hkv, Dv, K = _check_shapes(q, k, v, idx)
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(Dqk)
    dq = torch.zeros(B, Sq, Hq, Dqk, dtype=dtype)
    dk = torch.zeros(B, Skv, Hkv, Dqk, dtype=dtype)
    dv = torch.zeros(B, Skv, Hkv, Dv, dtype=dtype)
    dsink = torch.zeros(Hq, dtype=dtype) if sink is not None else None
    valid = valid_mask(idx, Skv, kv_lens)
    C = _chunk_size(Sq, G, K, max(Dqk, Dv), torch.finfo(dtype).bits // 8, max_chunk_bytes)
    for b in range(B):
        for g in range(Hkv):
            kb = k[b, :, g].to(dtype)
            vb = v[b, :, g].to(dtype)
            for s0 in range(0, Sq, C):
                s1 = min(Sq, s0 + C)
                vm = valid[b, s0:s1, g]
                safe = torch.where(vm, idx[b, s0:s1, g].long(), torch.zeros_like(vm, dtype=torch.long))
                kg = _gather_rows(kb, safe)
                vg = _gather_rows(vb, safe)
                qg = q[b, s0:s1, g * G:(g + 1) * G].to(dtype)
                og = out[b, s0:s1, g * G:(g + 1) * G].to(dtype)
                dog = dout[b, s0:s1, g * G:(g + 1) * G].to(dtype)
                lg = lse[b, s0:s1, g * G:(g + 1) * G].to(dtype)
                lfin = torch.where(torch.isfinite(lg), lg, torch.zeros_like(lg))
                delta = (og * dog).sum(-1)                                  # [C, G]
                s = torch.einsum("cgd,ckd->cgk", qg, kg) * scale
                p = torch.exp(s - lfin[..., None])
                p = torch.where(vm[:, None, :], p, torch.zeros_like(p))     # SFA.py:696
                dp = torch.einsum("cgd,ckd->cgk", dog, vg)                 # SFA.py:679
                ds = p * (dp - delta[..., None])                            # SFA.py:697-698
                dq[b, s0:s1, g * G:(g + 1) * G] = scale * torch.einsum("cgk,ckd->cgd", ds, kg)
                dk_c = scale * torch.einsum("cgk,cgd->ckd", ds, qg)         # SFA.py:841-846
                dv_c = torch.einsum("cgk,cgd->ckd", p, dog)                 # SFA.py:831
                w = vm.reshape(-1)
                flat = safe.reshape(-1)[w]
                dk[b, :, g].index_add_(0, flat, dk_c.reshape(-1, Dqk)[w])   # SFA.py:853
                dv[b, :, g].index_add_(0, flat, dv_c.reshape(-1, Dv)[w])
                if sink is not None:
                    sg = sink[g * G:(g + 1) * G].to(dtype)
                    psink = torch.where(torch.isfinite(lg), torch.exp(sg[None, :] - lfin), torch.zeros_like(lg))
                    dsink[g * G:(g + 1) * G] -= (psink * delta).sum(0)
    return dq, dk, dv, dsink


def sfa_forward_autograd(q, k, v, idx, scale=None, kv_lens=None, sink=None):
    """Differentiable dense restatement (no chunking) for ``gradcheck`` and for
    checking ``sfa_backward`` against autograd; small inputs only."""
    B, Sq, Hq, Dqk, Skv, Hkv, Dv, K = _check_shapes(q, k, v, idx)
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(Dqk)
    valid = valid_mask(idx, Skv, kv_lens)
    safe = torch.where(valid, idx.long(), torch.zeros_like(idx, dtype=torch.long))
    outs, lses = [], []
    for b in range(B):
        ob, lb = [], []
        for g in range(Hkv):
            vm = valid[b, :, g]
            kg = k[b, :, g][safe[b, :, g]]
            vg = v[b, :, g][safe[b, :, g]]
            qg = q[b, :, g * G:(g + 1) * G]
            s = torch.einsum("sgd,skd->sgk", qg, kg) * scale
            s = s.masked_fill(~vm[:, None, :], -math.inf)
            if sink is not None:
                sk = sink[g * G:(g + 1) * G].view(1, G, 1).expand(s.shape[0], G, 1)
                s_all = torch.cat([s, sk], dim=-1)
                l = torch.logsumexp(s_all, dim=-1)
                p = torch.softmax(s_all, dim=-1)[..., :-1]
            else:
                l = torch.logsumexp(s, dim=-1)
                p = torch.softmax(s, dim=-1)
                p = torch.nan_to_num(p, nan=0.0)
            ob.append(torch.einsum("sgk,skd->sgd", p, vg))
            lb.append(l)
        outs.append(torch.cat(ob, dim=1))
        lses.append(torch.cat(lb, dim=1))
    return torch.stack(outs), torch.stack(lses)


def paged_to_contiguous(k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                        idx: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Contiguous ``(k, v, idx)`` equivalent to a paged cache.

    ``k_cache`` / ``v_cache``: ``[num_pages, page_size, Hkv, D]`` pools;
    ``block_table``: ``[B, max_pages]`` pool page of each logical page;
    ``idx``: ``[B, Sq, Hkv, K]`` logical key positions.  Returns
    ``k``/``v`` ``[B, max_pages * page_size, Hkv, D]`` (rows of unmapped pages
    are zero) and ``idx`` with every slot whose page is unmapped set to -1
    (other slots unchanged, so the range / ``kv_lens`` rules still apply).
    """
    num_pages, page_size = k_cache.shape[:2]
    B, max_pages = block_table.shape
    bt = block_table.long()
    mapped = (bt >= 0) & (bt < num_pages)                       # [B, max_pages]
    safe = torch.where(mapped, bt, torch.zeros_like(bt))

    def gather(cache):
        rows = cache[safe.reshape(-1)]                           # [B*max_pages, page, Hkv, D]
        rows = rows * mapped.reshape(-1, 1, 1, 1).to(rows.dtype)
        return rows.reshape(B, max_pages * page_size, *cache.shape[2:])

    il = idx.long()
    page = torch.div(il, page_size, rounding_mode="floor")
    in_table = (il >= 0) & (page < max_pages)
    pmapped = torch.gather(mapped, 1, torch.where(in_table, page, torch.zeros_like(page)).reshape(B, -1))
    pmapped = pmapped.reshape(idx.shape) & in_table
    idx_out = torch.where(pmapped | (il < 0) | ~in_table, idx, torch.full_like(idx, -1))
    return gather(k_cache), gather(v_cache), idx_out




def indexer_key_end(B: int, Sq: int, Skv: int, kv_lens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``[B, Sq]`` int64: query t of sequence b may see keys ``[0, end)``,
    ``end = clamp(t + 1 + L_b - Sq, 0, L_b)``, ``L_b = min(kv_lens[b], Skv)`` or ``Skv``."""
    L = torch.full((B,), Skv, dtype=torch.int64) if kv_lens is None else kv_lens.long().cpu().clamp(max=Skv)
    t = torch.arange(Sq, dtype=torch.int64)
    end = t[None, :] + 1 + L[:, None] - Sq
    return torch.minimum(end, L[:, None]).clamp(min=0)


def indexer_scores(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, kv_lens: Optional[torch.Tensor] = None,
                   dtype: torch.dtype = torch.float32, max_chunk_bytes: int = 1 << 28,
                   k_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Lightning-indexer scores ``[B, Sq, Skv]``: ``sum_h w * relu(<q_h, k_s>)``
    for the keys each query may see, ``-inf`` elsewhere.  ``q`` ``[B, Sq, H, D]``,
    ``k`` ``[B, Skv, D]`` (bf16, fp32 or fp8 e4m3: every element is exact in
    ``dtype``), ``w`` ``[B, Sq, H]``; ``k_scale`` ``[B, Skv]`` (positive) scales
    the keys' scores, as DeepSeek-V3.2's fp8 indexer does."""
    B, Sq, H, D = q.shape
    Skv = k.shape[1]
    end = indexer_key_end(B, Sq, Skv, kv_lens)
    out = torch.empty(B, Sq, Skv, dtype=dtype)
    rows = max(1, max_chunk_bytes // max(1, H * Skv * torch.finfo(dtype).bits // 8))
    pos = torch.arange(Skv)
    for b in range(B):
        kb = k[b].to(dtype)
        for t0 in range(0, Sq, rows):
            t1 = min(Sq, t0 + rows)
            dots = torch.einsum("thd,sd->ths", q[b, t0:t1].to(dtype), kb)
            sc = torch.einsum("th,ths->ts", w[b, t0:t1].to(dtype), dots.clamp_min(0))
            if k_scale is not None:
                sc = sc * k_scale[b].to(dtype)[None, :]
            allowed = pos[None, :] < end[b, t0:t1, None]
            out[b, t0:t1] = torch.where(allowed, sc, torch.full_like(sc, -math.inf))
    return out


def indexer_topk(scores: torch.Tensor, topk: int, end: torch.Tensor) -> torch.Tensor:
    """``[B, Sq, 1, topk]`` int32 from scores ``[B, Sq, Skv]`` and the per-row
    key ends ``[B, Sq]``: rows with ``end <= topk`` keep every allowed key;
    others the ``topk`` keys of largest score, equal scores ordered by key
    (a stable sort of descending scores); both in ascending key order, then -1."""
    B, Sq, Skv = scores.shape
    out = torch.full((B, Sq, 1, topk), -1, dtype=torch.int32)
    for b in range(B):
        for t in range(Sq):
            n = int(end[b, t])
            if n <= topk:
                sel = torch.arange(n)
            else:
                order = torch.sort(scores[b, t, :n], descending=True, stable=True).indices
                sel = torch.sort(order[:topk]).values
            out[b, t, 0, :sel.numel()] = sel.to(torch.int32)
    return out
