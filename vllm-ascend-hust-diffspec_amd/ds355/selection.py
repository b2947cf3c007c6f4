"""Top-k chunk selection on MI355X — drop-in for ``diffspec.runtime.select_context_chunks``.

``select_context_chunks`` keeps the reference's signature, checks and result
type (diffspec/runtime.py:44-48, 348-414) and runs the HIP kernel
``ds_select_chunks``; ``select_context_chunks_batched`` selects for a whole
batch in one launch (the reference loops over rows, runtime.py:1298-1308).
Equal scores are ordered by the lower chunk index.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class DiffSpecSelection:
    chunk_indices: torch.Tensor
    token_indices: torch.Tensor
    chunk_scores: torch.Tensor


def selection_capacity(history_budget: int, chunk_size: int) -> int:
    """Chunks kept per request, including the forced newest chunk."""
    return history_budget // chunk_size


def select_context_chunks_batched(
    chunk_scores: torch.Tensor,
    seq_lens: torch.Tensor,
    chunk_size: int,
    history_budget: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """One launch over ``[B, >= max chunks]`` fp32 scores.

    Returns ``(ids [B, history_budget // chunk_size] int32, counts [B] int32)``;
    row b's ids are ``ids[b, :counts[b]]``, ascending.
    """
    if chunk_scores.ndim != 2:
        raise ValueError("chunk_scores must be two-dimensional")
    if chunk_size <= 0 or history_budget < chunk_size or history_budget % chunk_size != 0:
        raise ValueError("token_budget must be a positive chunk-size multiple")
    device = _lib.require_gpu(chunk_scores, seq_lens)
    scores = chunk_scores if chunk_scores.dtype == torch.float32 else chunk_scores.float()
    if scores.stride(1) != 1:
        scores = scores.contiguous()
    lens = (seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)).contiguous()
    batch = scores.shape[0]
    capacity = selection_capacity(history_budget, chunk_size)
    ids = torch.zeros((batch, capacity), dtype=torch.int32, device=device)
    counts = torch.zeros((batch,), dtype=torch.int32, device=device)
    lib = _lib.load()
    _lib.check(lib.ds_select_chunks(
        _lib.stream_handle(device), scores.data_ptr(), scores.stride(0), scores.shape[1], lens.data_ptr(), batch,
        chunk_size, history_budget, ids.data_ptr(), ids.stride(0), counts.data_ptr(),
    ))
    return ids, counts


def select_context_chunks(
    chunk_scores: torch.Tensor,
    seq_len: int,
    chunk_size: int,
    token_budget: int,
) -> DiffSpecSelection:
    """Select top scoring chunks while always retaining the newest chunk.

    ``token_budget`` is the selection capacity (the caller's history budget,
    runtime.py:1560-1565).  No device value is read back: the number of
    selected chunks, ``min(ceil(seq_len / chunk), token_budget // chunk)``, is
    known on the host.
    """
    if chunk_scores.ndim != 1:
        raise ValueError("chunk_scores must be one-dimensional")
    if seq_len < 0:
        raise ValueError("seq_len must be non-negative")
    if token_budget < chunk_size or token_budget % chunk_size != 0:
        raise ValueError("token_budget must be a positive chunk-size multiple")
    num_chunks = (seq_len + chunk_size - 1) // chunk_size
    if num_chunks != chunk_scores.numel():
        raise ValueError("chunk score count does not match sequence length")
    device = _lib.require_gpu(chunk_scores)
    if num_chunks == 0:
        empty = torch.empty(0, dtype=torch.long, device=device)
        return DiffSpecSelection(empty, empty, chunk_scores)
    lens = torch.full((1,), seq_len, dtype=torch.int32, device=device)
    ids, _ = select_context_chunks_batched(chunk_scores.reshape(1, -1), lens, chunk_size, token_budget)
    count = min(num_chunks, token_budget // chunk_size)
    selected = ids[0, :count].long()
    offsets = torch.arange(chunk_size, dtype=torch.long, device=device)
    if seq_len % chunk_size:
        full = (selected[:-1, None] * chunk_size + offsets[None, :]).reshape(-1)
        tail = torch.arange((num_chunks - 1) * chunk_size, seq_len, dtype=torch.long, device=device)
        tokens = torch.cat((full, tail))
    else:
        tokens = (selected[:, None] * chunk_size + offsets[None, :]).reshape(-1)
    return DiffSpecSelection(selected, tokens, chunk_scores.index_select(0, selected))
