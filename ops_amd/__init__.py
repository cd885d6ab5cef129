"""ops_amd — MI355X (gfx950) top-k sparse flash attention.

Public API (BSHD, see ``ops_amd.sfa``)::

    out, lse = ops_amd.sparse_flash_attention(q, k, v, topk_idxs, sm_scale=None,
                                              kv_lens=None, attn_sink=None)

Paged KV cache (serving): ``ops_amd.sfa_forward_paged(q, k_cache, v_cache,
block_table, topk_idxs, ...)``.

Top-k index producer (scores + selection that create ``topk_idxs``):
``ops_amd.indexer_topk(q_idx, k_idx, weights, topk, kv_lens=None)``.

The HIP kernels live in ``libsfa.so`` (``python -m ops_amd.build``), reached
through the C ABI declared in ``include/sfa.h``.
"""
from .indexer import indexer_topk
from .sfa import (SparseFlashAttention, SparseFlashAttentionSBHD, SparseFlashAttentionTriton, sfa_backward,
                  sfa_forward, sfa_forward_paged, sparse_flash_attention)

__all__ = ["SparseFlashAttention", "sparse_flash_attention", "sfa_forward", "sfa_backward", "sfa_forward_paged",
           "SparseFlashAttentionSBHD", "SparseFlashAttentionTriton", "indexer_topk"]
