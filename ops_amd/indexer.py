"""Top-k index producer on MI355X: scores + top-k selection that create the
``topk_idxs`` rows the sparse attention consumes.

The reference takes the index rows as an input (``topk_idxs``: "Sparse
indices mapping queries to KV blocks", lilac-me/ops SFA.py:88-90).  The
scores are DeepSeek-V3.2's lightning indexer::

    I[b, t, s] = sum_h w[b, t, h] * relu(<q[b, t, h, :], k[b, s, :]>)

over the keys a query may see (``s <= t + L_b - Sq`` with ``L_b = kv_lens[b]``
or ``Skv``); each row keeps the ``topk`` best keys (equal scores: the lower key
first) in ascending key order, then ``-1`` padding.  Both steps run as HIP
kernels of ``libsfa.so`` (``sfa_indexer_topk``, ``include/sfa.h``).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

__all__ = ["indexer_topk"]


def indexer_topk(q: torch.Tensor, k: torch.Tensor, weights: torch.Tensor, topk: int,
                 kv_lens: Optional[torch.Tensor] = None, return_logits: bool = False,
                 k_scale: Optional[torch.Tensor] = None):
    """``q`` ``[B, Sq, H, 128]``, ``k`` ``[B, Skv, 128]`` (one index key per
    token), both bfloat16 or both float8_e4m3fn, ``weights`` ``[B, Sq, H]``
    (float32 after conversion; with fp8, the q scales folded in).  ``k_scale``
    ``[B, Skv]`` (fp8 only, positive): the score of key s is multiplied by it.

    Returns ``topk_idxs`` ``[B, Sq, 1, topk]`` int32, ready for
    :func:`ops_amd.sparse_flash_attention` with one KV head, and with
    ``return_logits`` also the scores ``[B, Sq, Skv]`` float32 (entries of keys
    a query may not see are unspecified).
    """
    lib = _lib.load()
    if q.dim() != 4 or k.dim() != 3 or weights.dim() != 3:
        raise ValueError("expected q [B, Sq, H, D], k [B, Skv, D], weights [B, Sq, H]")
    B, Sq, H, D = q.shape
    if k.shape[0] != B or k.shape[2] != D or tuple(weights.shape) != (B, Sq, H):
        raise ValueError(f"shapes do not match: q {tuple(q.shape)}, k {tuple(k.shape)}, weights {tuple(weights.shape)}")
    for name, t in (("q", q), ("k", k), ("weights", weights)):
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be a GPU tensor (got device {t.device})")
    f8 = getattr(torch, "float8_e4m3fn", None)
    if q.dtype != k.dtype or q.dtype not in (torch.bfloat16, f8):
        raise ValueError("q and k must both be bfloat16 or both float8_e4m3fn")
    fp8 = q.dtype == f8
    if k_scale is not None:
        if not fp8:
            raise ValueError("k_scale is for float8 keys only")
        if tuple(k_scale.shape) != (B, k.shape[1]) or k_scale.device != q.device:
            raise ValueError("k_scale must be a [B, Skv] tensor on q's device")
        k_scale = k_scale.to(torch.float32).contiguous()
    if int(topk) <= 0:
        raise ValueError(f"topk must be positive, got {topk}")
    Skv = k.shape[1]
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    w = weights.to(torch.float32)
    if w.stride(-1) != 1:
        w = w.contiguous()
    if kv_lens is not None:
        if kv_lens.numel() != B or kv_lens.device != q.device:
            raise ValueError("kv_lens must be a [B] tensor on q's device")
        kv_lens = kv_lens.to(torch.int32).contiguous()
    idx = torch.empty((B, Sq, 1, int(topk)), dtype=torch.int32, device=q.device)
    logits = None
    if return_logits:
        ld = (Skv + 3) // 4 * 4
        logits = torch.empty((B, Sq, ld), dtype=torch.float32, device=q.device)[..., :Skv]
    a = _lib.IndexerArgs()
    a.B, a.Sq, a.Skv, a.H, a.D, a.topk = B, Sq, Skv, H, D, int(topk)
    a.dtype = _lib.SFA_DTYPE_FP8_E4M3 if fp8 else _lib.SFA_DTYPE_BF16
    if k_scale is not None:
        a.k_scale, a.ks_sb = k_scale.data_ptr(), k_scale.stride(0)
    a.q, (a.q_sb, a.q_ss, a.q_sh) = q.data_ptr(), q.stride()[:3]
    a.k, (a.k_sb, a.k_ss) = k.data_ptr(), k.stride()[:2]
    a.w, (a.w_sb, a.w_ss) = w.data_ptr(), w.stride()[:2]
    a.kv_lens = kv_lens.data_ptr() if kv_lens is not None else None
    a.idx, a.i_sb, a.i_ss = idx.data_ptr(), idx.stride(0), idx.stride(1)
    if logits is not None:
        a.logits, (a.g_sb, a.g_ss) = logits.data_ptr(), logits.stride()[:2]
    a.flags = 0
    ws = lib.sfa_indexer_topk_workspace_size(ctypes.byref(a))
    wbuf = torch.empty(ws, dtype=torch.uint8, device=q.device) if ws else None
    stream = torch.cuda.current_stream(q.device).cuda_stream
    _lib.check(lib.sfa_indexer_topk(ctypes.byref(a), None if wbuf is None else ctypes.c_void_p(wbuf.data_ptr()), ws,
                                    ctypes.c_void_p(stream)))
    return (idx, logits) if return_logits else idx
