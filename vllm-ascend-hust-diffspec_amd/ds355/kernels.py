"""Paged chunk scores on MI355X — drop-in for ``diffspec.kernels``.

``paged_chunk_attention_scores`` keeps the signature, argument meaning,
output and ``ValueError`` messages of diffspec/kernels.py:95-150; the Triton
kernel is replaced by the HIP kernel ``ds_chunk_scores`` (one streaming pass
over K that multiplies each key row by all query heads of its GQA group and
fuses the head mean).  ``softmax_lse=None`` (not in the reference kernel)
gives the reference's ``chunk_attention_scores`` without an LSE
(diffspec/runtime.py:321-322): each head is normalised over the row's own
scored tokens, computed in the same single pass over K.
"""

from __future__ import annotations

import torch

from . import _lib


def paged_chunk_attention_scores(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    softmax_lse: torch.Tensor | None,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    chunk_size: int,
    max_seq_len: int,
    scale: float,
    head_reduce: str = "mean",
) -> torch.Tensor:
    """Compute normalized logical-chunk attention scores from paged K.

    query ``[B, Hq, D]``, key_cache ``[blocks, block_size, Hkv, D]`` (bf16 or
    fp16), softmax_lse with ``B * Hq`` values, block_table ``[B, max_blocks]``
    and seq_lens ``[B]`` -> fp32 ``[B, ceil(max_seq_len / chunk_size)]``;
    chunks past a row's length are 0.  ``head_reduce="max"`` (not in the
    reference) takes the largest weight over heads per token instead of the
    head mean.  ``softmax_lse=None`` normalises each head over the row's own
    tokens (head mean only).
    """
    if query.ndim != 3:
        raise ValueError("query must have shape [batch, query_heads, head_dim]")
    if key_cache.ndim != 4:
        raise ValueError("key_cache must have shape [blocks, block_size, kv_heads, head_dim]")
    batch_size, num_query_heads, head_dim = query.shape
    _, block_size, num_kv_heads, key_head_dim = key_cache.shape
    if head_dim != key_head_dim:
        raise ValueError("query and key head dimensions must match")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("query heads must be divisible by KV heads")
    if softmax_lse is not None and softmax_lse.numel() != batch_size * num_query_heads:
        raise ValueError("softmax_lse must contain one value per query head")
    if softmax_lse is None and head_reduce != "mean":
        raise ValueError("head_reduce='max' needs a supplied softmax_lse")
    if head_reduce not in ("mean", "max"):
        raise ValueError("head_reduce must be 'mean' or 'max'")
    if query.dtype != key_cache.dtype:
        raise ValueError("query and key cache must share a dtype")
    device = _lib.require_gpu(query, key_cache, softmax_lse, block_table, seq_lens)
    lib = _lib.load()

    max_chunks = (max_seq_len + chunk_size - 1) // chunk_size if chunk_size > 0 else 0
    out = torch.empty((batch_size, max_chunks), dtype=torch.float32, device=device)
    if query.stride(2) != 1 or query.stride(1) != head_dim:
        query = query.contiguous()
    if key_cache.stride(3) != 1:
        key_cache = key_cache.contiguous()
    lse = None
    if softmax_lse is not None:
        lse = softmax_lse.reshape(batch_size, num_query_heads)
        if lse.dtype != torch.float32:
            lse = lse.float()
    table = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    if table.ndim != 2 or table.stride(1) != 1:
        table = table.reshape(batch_size, -1).contiguous()
    lens = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
    lens = lens.contiguous()
    mode = _lib.DS_HEAD_MAX if head_reduce == "max" else _lib.DS_HEAD_MEAN
    workspace = None
    if mode == _lib.DS_HEAD_MEAN:
        # Per-KV-head partials; without an LSE, preceded by a (max, sum) pair
        # per (query head, chunk) and each row's head LSEs.
        size = batch_size * max_chunks * num_kv_heads
        if lse is None:
            size += batch_size * (max_chunks * 2 * num_query_heads + num_query_heads)
        workspace = torch.empty(size, dtype=torch.float32, device=device)
    _lib.check(lib.ds_chunk_scores(
        _lib.stream_handle(device), _lib.dtype_code(query.dtype),
        query.data_ptr(), query.stride(0),
        key_cache.data_ptr(), key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
        _lib.ptr(lse), 0 if lse is None else lse.stride(0), 0 if lse is None else lse.stride(1),
        table.data_ptr(), table.stride(0),
        lens.data_ptr(),
        batch_size, num_query_heads, num_kv_heads, head_dim, block_size, chunk_size, max_chunks,
        float(scale), mode, out.data_ptr(), out.stride(0),
        _lib.ptr(workspace), 0 if workspace is None else workspace.numel() * 4,
    ))
    return out
