"""Top-k sparse flash attention on MI355X: the drop-in host layer.

Reference: ``SparseFlashAttentionTriton`` (lilac-me/ops SFA.py:69-306), an
autograd Function whose forward launches ``_attn_fwd`` and whose backward
launches ``_attn_bwd_dq_dsink`` and ``_attn_bwd_dk_dv``.  This module keeps
that role and calls the HIP kernels of ``libsfa.so`` through its C ABI
(``include/sfa.h``) on torch's current stream:

``SparseFlashAttention.apply(q, k, v, topk_idxs, sm_scale, kv_lens, attn_sink)``
    -> ``(out, lse)``; backward returns ``dq, dk, dv`` (and ``dsink``).

Layout is BSHD: q ``[B, Sq, Hq, Dqk]``, k ``[B, Skv, Hkv, Dqk]``,
v ``[B, Skv, Hkv, Dv]`` (``v`` may be a view of ``k``, e.g. MLA's
``kv[..., :512]``), topk_idxs ``[B, Sq, Hkv, K]`` int32 with -1 padding,
``lse`` float32 natural log ``[B, Sq, Hq]``.  Query head ``h`` reads KV head
``h // (Hq // Hkv)``.  A slot is valid iff ``0 <= idx < kv_lens[b]`` (or
``Skv``); invalid slots contribute nothing, at any slot position.

Error behaviour follows the reference: an empty index tensor or a
non-positive top-k raises ``ValueError`` (SFA.py:52-53, 63-64); this layer
also raises ``ValueError`` for device/dtype/shape mismatches the reference
leaves unchecked.  There is no host synchronisation (the reference's
``_effective_topk`` ``.item()``, SFA.py:62-66, is replaced by device-side
masking of every slot), so the op can be captured in a HIP graph.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Tuple

import torch

from . import _lib

__all__ = ["SparseFlashAttention", "sparse_flash_attention", "sfa_forward", "sfa_backward", "sfa_forward_paged",
           "SparseFlashAttentionSBHD", "SparseFlashAttentionTriton"]

_DTYPES = {torch.float32: _lib.SFA_DTYPE_F32, torch.bfloat16: _lib.SFA_DTYPE_BF16}
_DKV_MODES = {"auto": _lib.SFA_DKV_AUTO, "atomic": _lib.SFA_DKV_ATOMIC, "csr": _lib.SFA_DKV_CSR}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _rows(t: torch.Tensor) -> torch.Tensor:
    """The kernels need a unit stride on the feature dimension."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _validate(q, k, v, idx, kv_lens, sink):
    if idx.numel() == 0:  # SFA.py:63-64
        raise ValueError("topk_idxs tensor is empty. Cannot determine effective topk.")
    for name, t in (("q", q), ("k", k), ("v", v), ("topk_idxs", idx)):
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4-D (BSHD), got shape {tuple(t.shape)}")
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be a GPU tensor (got device {t.device})")
    if not (q.device == k.device == v.device == idx.device):
        raise ValueError("q, k, v, topk_idxs must be on the same device")
    if q.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {q.dtype}; expected bfloat16 or float32")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share one dtype")
    B, Sq, Hq, Dqk = q.shape
    Bk, Skv, Hkv, Dk = k.shape
    if Bk != B or Dk != Dqk:
        raise ValueError(f"k shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if tuple(v.shape[:3]) != (B, Skv, Hkv):
        raise ValueError(f"v shape {tuple(v.shape)} does not match k {tuple(k.shape)}")
    if Hq % Hkv != 0:
        raise ValueError(f"Hq ({Hq}) must be a multiple of Hkv ({Hkv})")
    if tuple(idx.shape[:3]) != (B, Sq, Hkv):
        raise ValueError(f"topk_idxs must be [B, Sq, Hkv, K] = [{B}, {Sq}, {Hkv}, K], got {tuple(idx.shape)}")
    if idx.shape[3] <= 0:  # SFA.py:52-53
        raise ValueError(f"Unsupported topk value: {idx.shape[3]}. Please make sure it is a positive integer.")
    if kv_lens is not None and (kv_lens.numel() != B or kv_lens.device != q.device):
        raise ValueError("kv_lens must be a [B] tensor on q's device")
    if sink is not None and (sink.numel() != Hq or sink.device != q.device):
        raise ValueError("attn_sink must be a [Hq] tensor on q's device")


def _fwd_args(q, k, v, idx, out, lse, scale, kv_lens, sink, num_splits, idx_sorted=False) -> _lib.FwdArgs:
    B, Sq, Hq, Dqk = q.shape
    _, Skv, Hkv, _ = k.shape
    a = _lib.FwdArgs()
    a.dtype = _DTYPES[q.dtype]
    a.B, a.Sq, a.Skv, a.Hq, a.Hkv = B, Sq, Skv, Hq, Hkv
    a.Dqk, a.Dv, a.topk = Dqk, v.shape[3], idx.shape[3]
    a.scale = float(scale)
    a.q, (a.q_sb, a.q_ss, a.q_sh) = q.data_ptr(), q.stride()[:3]
    a.k, (a.k_sb, a.k_ss, a.k_sh) = k.data_ptr(), k.stride()[:3]
    a.v, (a.v_sb, a.v_ss, a.v_sh) = v.data_ptr(), v.stride()[:3]
    a.idx, (a.i_sb, a.i_ss, a.i_sh) = idx.data_ptr(), idx.stride()[:3]
    a.kv_lens = kv_lens.data_ptr() if kv_lens is not None else None
    a.sink = sink.data_ptr() if sink is not None else None
    a.out, (a.o_sb, a.o_ss, a.o_sh) = out.data_ptr(), out.stride()[:3]
    a.lse, (a.l_sb, a.l_ss, a.l_sh) = lse.data_ptr(), lse.stride()
    a.num_splits = int(num_splits)
    a.flags = _lib.SFA_FWD_IDX_SORTED if idx_sorted else 0
    return a


def _prep(q, k, v, topk_idxs, kv_lens, sink, validate=True):
    if validate:
        _validate(q, k, v, topk_idxs, kv_lens, sink)
    q, k, v = _rows(q), _rows(k), _rows(v)
    idx = topk_idxs
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
    if kv_lens is not None:
        kv_lens = kv_lens.to(torch.int32).contiguous()
    if sink is not None:
        sink = sink.to(torch.float32).contiguous()
    return q, k, v, idx, kv_lens, sink


def sfa_forward(q, k, v, topk_idxs, sm_scale=None, kv_lens=None, attn_sink=None, num_splits: int = 0,
                out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None, noalloc: bool = False,
                idx_sorted: bool = False):
    """Forward only (no autograd): ``(out, lse)``.  ``out``/``lse`` may be
    preallocated ([B, Sq, Hq, Dv] in q's dtype / [B, Sq, Hq] float32).
    ``noalloc=True`` calls ``sfa_fwd_noalloc``: the split-k partials then live
    in the library's static per-GPU scratch (64 MiB) instead of a workspace
    tensor, so with preallocated ``out``/``lse`` nothing is allocated.
    ``idx_sorted=True`` declares every index row ascending before its padding
    (as :func:`ops_amd.indexer.indexer_topk` writes them): the MLA prefill
    then skips the pass that sorts them (``SFA_FWD_IDX_SORTED``)."""
    lib = _lib.load()
    q, k, v, idx, kv_lens, sink = _prep(q, k, v, topk_idxs, kv_lens, attn_sink)
    B, Sq, Hq, Dqk = q.shape
    Dv = v.shape[3]
    scale = (1.0 / math.sqrt(Dqk)) if sm_scale is None else float(sm_scale)
    if out is None:
        out = torch.empty((B, Sq, Hq, Dv), dtype=q.dtype, device=q.device)
    if lse is None:
        lse = torch.empty((B, Sq, Hq), dtype=torch.float32, device=q.device)
    a = _fwd_args(q, k, v, idx, out, lse, scale, kv_lens, sink, num_splits, idx_sorted)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    if noalloc:
        _lib.check(lib.sfa_fwd_noalloc(ctypes.byref(a), ctypes.c_void_p(stream)))
        return out, lse
    ws = lib.sfa_fwd_workspace_size(ctypes.byref(a))
    wbuf = torch.empty(ws, dtype=torch.uint8, device=q.device) if ws else None
    _lib.check(lib.sfa_fwd(ctypes.byref(a), _ptr(wbuf), ws, ctypes.c_void_p(stream)))
    return out, lse


def sfa_forward_paged(q, k_cache, v_cache, block_table, topk_idxs, sm_scale=None, kv_lens=None, attn_sink=None,
                      num_splits: int = 0, out: Optional[torch.Tensor] = None,
                      lse: Optional[torch.Tensor] = None):
    """Forward over a paged KV cache (no autograd): ``(out, lse)``.

    ``k_cache`` ``[num_pages, page_size, Hkv, Dqk]`` and ``v_cache``
    ``[num_pages, page_size, Hkv, Dv]`` are page pools (``v_cache`` may be a
    view of ``k_cache``, e.g. MLA's ``k_cache[..., :512]``); ``block_table``
    ``[B, max_pages]`` int32 maps page ``i // page_size`` of sequence ``b`` to
    a pool page; ``topk_idxs`` ``[B, Sq, Hkv, K]`` hold *logical* key
    positions, valid iff ``0 <= idx < kv_lens[b]`` (or
    ``max_pages * page_size``) and mapped to a page in ``[0, num_pages)``.
    The result equals :func:`sfa_forward` on the contiguous cache the block
    table describes.  ``page_size`` must be a power of two.
    """
    lib = _lib.load()
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("k_cache / v_cache must be [num_pages, page_size, Hkv, D]")
    if block_table.dim() != 2 or block_table.shape[0] != q.shape[0]:
        raise ValueError(f"block_table must be [B, max_pages] with B = {q.shape[0]}")
    if block_table.device != q.device:
        raise ValueError("block_table must be on q's device")
    num_pages, page_size, Hkv, _ = k_cache.shape
    if tuple(v_cache.shape[:3]) != (num_pages, page_size, Hkv):
        raise ValueError(f"v_cache shape {tuple(v_cache.shape)} does not match k_cache {tuple(k_cache.shape)}")
    if page_size <= 0 or page_size & (page_size - 1):
        raise ValueError(f"page_size must be a power of two, got {page_size}")
    max_pages = block_table.shape[1]
    B = q.shape[0]
    skv = max_pages * page_size
    # stand-ins of the logical [B, Skv, Hkv, D] caches for the shared
    # validation (zero-stride; the library gets the pools' strides)
    kview = k_cache.new_empty(()).expand(B, skv, Hkv, k_cache.shape[3])
    vview = v_cache.new_empty(()).expand(B, skv, Hkv, v_cache.shape[3])
    _validate(q, kview, vview, topk_idxs, kv_lens, attn_sink)
    q, k_cache, v_cache, idx, kv_lens, sink = _prep(q, k_cache.unsqueeze(0), v_cache.unsqueeze(0), topk_idxs,
                                                    kv_lens, attn_sink, validate=False)
    k_cache, v_cache = k_cache.squeeze(0), v_cache.squeeze(0)
    bt = block_table.to(torch.int32)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    B, Sq, Hq, Dqk = q.shape
    Dv = v_cache.shape[3]
    scale = (1.0 / math.sqrt(Dqk)) if sm_scale is None else float(sm_scale)
    if out is None:
        out = torch.empty((B, Sq, Hq, Dv), dtype=q.dtype, device=q.device)
    if lse is None:
        lse = torch.empty((B, Sq, Hq), dtype=torch.float32, device=q.device)
    a = _fwd_args(q, kview, vview, idx, out, lse, scale, kv_lens, sink, num_splits)
    # pools: page, row and head strides
    a.k, (a.k_sb, a.k_ss, a.k_sh) = k_cache.data_ptr(), k_cache.stride()[:3]
    a.v, (a.v_sb, a.v_ss, a.v_sh) = v_cache.data_ptr(), v_cache.stride()[:3]
    pg = _lib.KvPages()
    pg.block_table = bt.data_ptr()
    pg.bt_sb = bt.stride(0)
    pg.max_pages, pg.page_size, pg.num_pages, pg.flags = max_pages, page_size, num_pages, 0
    ws = lib.sfa_fwd_paged_workspace_size(ctypes.byref(a), ctypes.byref(pg))
    wbuf = torch.empty(ws, dtype=torch.uint8, device=q.device) if ws else None
    stream = torch.cuda.current_stream(q.device).cuda_stream
    _lib.check(lib.sfa_fwd_paged(ctypes.byref(a), ctypes.byref(pg), _ptr(wbuf), ws, ctypes.c_void_p(stream)))
    return out, lse


def _is_prefix_view(k: torch.Tensor, v: torch.Tensor) -> bool:
    """v is the first v.shape[-1] dims of k's rows (same memory and strides)."""
    return (v.data_ptr() == k.data_ptr() and v.dim() == k.dim() == 4 and v.stride()[:3] == k.stride()[:3]
            and v.shape[:3] == k.shape[:3] and v.shape[3] <= k.shape[3] and v.stride(-1) == k.stride(-1))


def _merge_in_autograd(k: torch.Tensor, v: torch.Tensor, needs_k: bool, needs_v: bool) -> bool:
    """Whether the backward may return dK + dV as k's gradient and None for v.

    That is exact only when autograd itself would add v's gradient into the
    rows of k: v is k, or a view of k (or of k's own base) that autograd
    tracks, its memory is the first Dv dims of k's rows, and both inputs
    want a gradient.  An alias that autograd does not see (a detached view,
    a second leaf over the same storage) shares memory but not gradients."""
    if not (needs_k and needs_v and _is_prefix_view(k, v)):
        return False
    return v is k or v._base is k or (v._base is not None and v._base is k._base)


def sfa_backward(q, k, v, topk_idxs, out, lse, dout, sm_scale=None, kv_lens=None, attn_sink=None,
                 dlse: Optional[torch.Tensor] = None, dkv_mode: Optional[str] = None, merge_kv: bool = False,
                 dq: Optional[torch.Tensor] = None, dk: Optional[torch.Tensor] = None,
                 dv: Optional[torch.Tensor] = None):
    """Backward only (no autograd): ``(dq, dk, dv, dsink)``; ``dsink`` is None
    without a sink.  ``dq`` / ``dk`` / ``dv`` may be preallocated (q's / k's
    / v's shape and dtype, unit feature stride); they are fully overwritten.

    ``merge_kv=True`` (``v`` must be the first ``Dv`` dims of ``k``'s rows,
    e.g. MLA's ``kv[..., :512]``): ``dk`` is the gradient of the shared rows,
    dK + dV on their first ``Dv`` dims, as the reference sums both into one
    buffer (SFA.py:849-853), and ``dv`` is None.  The MLA shape (576 / 512,
    65..128 heads per KV head, bf16) then runs its MFMA backward."""
    lib = _lib.load()
    if merge_kv:
        if not _is_prefix_view(k, v):
            raise ValueError("merge_kv needs v to be the first Dv dims of k's rows (a prefix view of k)")
        _validate(q, k, v, topk_idxs, kv_lens, attn_sink)
        k = _rows(k)
        v = k[..., : v.shape[3]]
        q, k, v, idx, kv_lens, sink = _prep(q, k, v, topk_idxs, kv_lens, attn_sink, validate=False)
    else:
        q, k, v, idx, kv_lens, sink = _prep(q, k, v, topk_idxs, kv_lens, attn_sink)
    B, Sq, Hq, Dqk = q.shape
    _, Skv, Hkv, _ = k.shape
    Dv = v.shape[3]
    if tuple(dout.shape) != (B, Sq, Hq, Dv) or tuple(out.shape) != (B, Sq, Hq, Dv):
        raise ValueError("out / grad_out must be [B, Sq, Hq, Dv]")
    dout = _rows(dout.to(q.dtype))
    out = _rows(out)
    lse = lse.contiguous()
    scale = (1.0 / math.sqrt(Dqk)) if sm_scale is None else float(sm_scale)
    mode = dkv_mode or os.environ.get("SFA_DKV_MODE", "auto")
    if mode not in _DKV_MODES:
        raise ValueError(f"dkv_mode must be one of {sorted(_DKV_MODES)}")
    def _out(t, shape, name):
        if t is None:
            return torch.empty(shape, dtype=q.dtype, device=q.device)
        if tuple(t.shape) != shape or t.dtype != q.dtype or t.device != q.device or t.stride(-1) != 1:
            raise ValueError(f"{name} must be a {list(shape)} {q.dtype} tensor on {q.device} with a unit feature stride")
        return t

    dq = _out(dq, (B, Sq, Hq, Dqk), "dq")
    dk = _out(dk, (B, Skv, Hkv, Dqk), "dk")
    dv = None if merge_kv else _out(dv, (B, Skv, Hkv, Dv), "dv")
    dsink = torch.empty((Hq,), dtype=torch.float32, device=q.device) if sink is not None else None
    if dlse is not None:
        dlse = dlse.to(torch.float32).contiguous()
    a = _lib.BwdArgs()
    a.fwd = _fwd_args(q, k, v, idx, out, lse, scale, kv_lens, sink, 0)
    a.dout, (a.do_sb, a.do_ss, a.do_sh) = dout.data_ptr(), dout.stride()[:3]
    a.dq, (a.dq_sb, a.dq_ss, a.dq_sh) = dq.data_ptr(), dq.stride()[:3]
    a.dk, (a.dk_sb, a.dk_ss, a.dk_sh) = dk.data_ptr(), dk.stride()[:3]
    if dv is not None:
        a.dv, (a.dv_sb, a.dv_ss, a.dv_sh) = dv.data_ptr(), dv.stride()[:3]
    a.dlse = dlse.data_ptr() if dlse is not None else None
    a.dsink = dsink.data_ptr() if dsink is not None else None
    a.dkv_mode = _DKV_MODES[mode]
    a.flags = _lib.SFA_BWD_MERGE_KV if merge_kv else 0
    ws = lib.sfa_bwd_workspace_size(ctypes.byref(a))
    wbuf = torch.empty(ws, dtype=torch.uint8, device=q.device) if ws else None
    stream = torch.cuda.current_stream(q.device).cuda_stream
    _lib.check(lib.sfa_bwd(ctypes.byref(a), _ptr(wbuf), ws, ctypes.c_void_p(stream)))
    return dq, dk, dv, dsink


class SparseFlashAttention(torch.autograd.Function):
    """Autograd Function: ``apply(q, k, v, topk_idxs, sm_scale=None,
    kv_lens=None, attn_sink=None) -> (out, lse)``.

    Mirrors ``SparseFlashAttentionTriton`` (SFA.py:69-306) with the BSHD
    q/k/v API; ``sm_scale=None`` means ``1/sqrt(Dqk)`` in both directions
    (SFA.py:181-182).  The backward returns gradients for q, k, v and the
    sink; gradients reaching ``lse`` are honoured.
    """

    @staticmethod
    def forward(ctx, q, k, v, topk_idxs, sm_scale=None, kv_lens=None, attn_sink=None):
        out, lse = sfa_forward(q, k, v, topk_idxs, sm_scale, kv_lens, attn_sink)
        ctx.save_for_backward(q, k, v, topk_idxs, out, lse, kv_lens, attn_sink)
        ctx.sm_scale = sm_scale
        # decided here, where the inputs' autograd identity is still known
        ctx.merge_kv = _merge_in_autograd(k, v, ctx.needs_input_grad[1], ctx.needs_input_grad[2])
        ctx.mark_non_differentiable()
        ctx.set_materialize_grads(False)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        q, k, v, idx, out, lse, kv_lens, sink = ctx.saved_tensors
        if grad_out is None:
            grad_out = torch.zeros_like(out)
        # v an autograd view of k's first Dv dims (MLA's shared kv): the
        # merged gradient of the shared rows goes to k, nothing to v (autograd
        # would add v's gradient into the same rows of k)
        dq, dk, dv, dsink = sfa_backward(q, k, v, idx, out, lse, grad_out, ctx.sm_scale, kv_lens, sink,
                                         dlse=grad_lse, merge_kv=ctx.merge_kv)
        if dsink is not None and sink is not None:
            dsink = dsink.to(sink.dtype)
        return dq, dk, dv, None, None, None, dsink


def sparse_flash_attention(q, k, v, topk_idxs, sm_scale=None, kv_lens=None, attn_sink=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Functional form of :class:`SparseFlashAttention`."""
    return SparseFlashAttention.apply(q, k, v, topk_idxs, sm_scale, kv_lens, attn_sink)


class SparseFlashAttentionSBHD(torch.autograd.Function):
    """The reference's exact operator signature (SFA.py:69-164, 166-306):

    ``apply(q [S, B, H, D], kv [S_kv, B, D], attn_sink [H], topk_idxs [S, B, K],
    sm_scale) -> out [S, B, H, D]``; backward returns
    ``(grad_q, grad_kv, grad_sink, None, None)``.

    One KV head whose rows serve as both K and V (SFA.py:116); the index row of
    query t is shared by all heads (SFA.py:538).  The SBHD tensors are passed
    to the kernels as strided BSHD views, so nothing is copied; the gradient
    of the shared ``kv`` is dK + dV (the reference sums them into one buffer,
    SFA.py:849-853).  ``out`` and the gradients are allocated in the layout
    of the tensor they belong to, as the reference allocates them
    (``empty_like(q)``, ``zeros_like(q)``, ``zeros_like(kv)``, SFA.py:104,
    184-185: a contiguous ``q`` gives a contiguous ``out``), and the kernels
    write them through BSHD views.
    """

    @staticmethod
    def forward(ctx, q, kv, attn_sink, topk_idxs, sm_scale=None):
        if q.dim() != 4 or kv.dim() != 3 or topk_idxs.dim() != 3:
            raise ValueError("expected q [S, B, H, D], kv [S_kv, B, D], topk_idxs [S, B, K]")
        qb = q.permute(1, 0, 2, 3)
        kb = kv.permute(1, 0, 2).unsqueeze(2)
        idx = topk_idxs.permute(1, 0, 2).unsqueeze(2)
        out = _rows(torch.empty_like(q))
        _, lse = sfa_forward(qb, kb, kb, idx, sm_scale, attn_sink=attn_sink, out=out.permute(1, 0, 2, 3))
        ctx.save_for_backward(q, kv, attn_sink, topk_idxs, out, lse)
        ctx.sm_scale = sm_scale
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, kv, sink, topk_idxs, out, lse = ctx.saved_tensors
        qb = q.permute(1, 0, 2, 3)
        kb = kv.permute(1, 0, 2).unsqueeze(2)
        idx = topk_idxs.permute(1, 0, 2).unsqueeze(2)
        grad_q = _rows(torch.empty_like(q))
        grad_kv = _rows(torch.empty_like(kv))
        _, _, _, dsink = sfa_backward(qb, kb, kb, idx, out.permute(1, 0, 2, 3), lse, grad_out.permute(1, 0, 2, 3),
                                      ctx.sm_scale, attn_sink=sink, merge_kv=True, dq=grad_q.permute(1, 0, 2, 3),
                                      dk=grad_kv.permute(1, 0, 2).unsqueeze(2))
        if dsink is not None and sink is not None:
            dsink = dsink.to(sink.dtype)
        return grad_q, grad_kv, dsink, None, None


# The reference's class name, for call sites that import it by name.
SparseFlashAttentionTriton = SparseFlashAttentionSBHD
