"""Draft decode attention over the working cache (one HIP launch).

Mirror of the linear path of ``DiffSpecDraftCache.forward_attention``
(diffspec/runtime.py:2024-2077 on the CPU, :2079-2134 on the NPU, where one
fused-attention call reads the ``[slot, head, token_budget, head_dim]``
capacity view with ``actual_seq_lengths_kv = position + 1``).  One launch
writes each row's new key/value at its local position, advances the slot's
working length and attends over the row's valid prefix; output rows past
the batch are zero.  Slots may be in any order: the kernel addresses each
row's slot directly, so the reference's split between a contiguous slot
view and an ``index_select`` copy has no counterpart here (neither copies).
"""

from __future__ import annotations

import torch

from . import _lib

__all__ = [
    "attention_workspace_bytes",
    "new_attention_workspace",
    "attention_status",
    "attention_epoch",
    "draft_linear_attention",
]

STATUS_BAD_POSITION = 1
STATUS_PARTIAL_TIMEOUT = 2


def attention_workspace_bytes(batch_rows: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                              token_budget: int) -> int:
    """Bytes of the attention workspace for up to ``batch_rows`` rows."""
    return int(_lib.load().ds_draft_attention_workspace_bytes(batch_rows, num_q_heads, num_kv_heads, head_dim,
                                                              token_budget))


def new_attention_workspace(batch_rows: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                            token_budget: int, device: torch.device | str) -> torch.Tensor:
    """Zero-filled workspace (uint8); keep it and pass it to every launch on one stream."""
    size = attention_workspace_bytes(batch_rows, num_q_heads, num_kv_heads, head_dim, token_budget)
    if size <= 0:
        raise ValueError("attention workspace sizes must be positive and num_q_heads a multiple of num_kv_heads")
    return torch.zeros(size, dtype=torch.uint8, device=device)


def attention_status(workspace: torch.Tensor) -> int:
    """Status word (reads the device): bit 0 a row's slot or position was out
    of range, bit 1 the last workgroup's wait for the others' "seen" words
    expired (that launch did not advance the working lengths)."""
    return int(workspace[8:12].view(torch.int32).item())


def attention_epoch(workspace: torch.Tensor) -> int:
    """Launches completed on this workspace that had at least one pending row."""
    return int(workspace[0:4].view(torch.int32).item())


def _as_heads(t: torch.Tensor, rows: int, heads: int, head_dim: int, name: str) -> torch.Tensor:
    if t.dim() == 2 and t.shape[1] == heads * head_dim:
        t = t.view(t.shape[0], heads, head_dim)
    if t.dim() != 3 or t.shape[1] != heads or t.shape[2] != head_dim:
        raise ValueError(f"{name} must be [tokens, {heads}, {head_dim}] or [tokens, {heads * head_dim}]")
    if t.shape[0] < rows:
        raise RuntimeError("DiffSpec draft tensors omit active request rows")
    if t.stride(2) != 1:
        raise ValueError(f"{name} must be contiguous in head_dim")
    return t


def _int32_rows(values, rows: int, device: torch.device, name: str) -> torch.Tensor:
    if isinstance(values, torch.Tensor):
        t = values.reshape(-1)[:rows]
        if t.numel() < rows:
            raise ValueError(f"{name} has fewer entries than pending rows")
        if t.device != device:
            raise ValueError(f"{name} must be on {device}")
        return t.to(torch.int32).contiguous() if t.dtype != torch.int32 or not t.is_contiguous() else t
    return torch.tensor(list(values)[:rows], dtype=torch.int32, device=device)


def draft_linear_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    output: torch.Tensor,
    working_key: torch.Tensor,
    working_value: torch.Tensor,
    working_lens: torch.Tensor,
    slots,
    positions=None,
    *,
    scale: float,
    workspace: torch.Tensor,
    reuse: dict | None = None,
    reuse_key=None,
) -> torch.Tensor:
    """One linear draft-attention step for ``len(slots)`` rows.

    ``slots``: canonical slot per row (host list or int32 device tensor).
    ``positions``: local position per row (host list, device tensor, or
    ``None`` = each slot's current ``working_lens`` entry, read on the
    device).  ``query``/``output`` are ``[tokens, Hq, D]`` (or ``[tokens,
    Hq*D]``), ``key``/``value`` ``[tokens, Hkv, D]``, the working caches
    ``[slots, Hkv, token_budget, D]`` contiguous, ``working_lens`` int32.
    Returns ``output``.  ``reuse`` (a dict the caller keeps) holds validated
    launch arguments per layout: a later call whose tensors differ only in
    their addresses skips the checks.  ``reuse_key`` replaces the layout key
    computed here when the caller knows it: everything but the addresses of
    ``query``, ``key``, ``value`` and ``output`` must then be the same for
    one key.
    """
    sig = None
    reusable = reuse is not None and isinstance(slots, torch.Tensor) and (positions is None
                                                                          or isinstance(positions, torch.Tensor))
    if reusable and reuse_key is not None:
        sig = reuse_key
    elif reusable:
        sig = (query.shape, query.stride(), key.shape, key.stride(), value.shape, value.stride(), output.shape,
               output.stride(), query.dtype, key.dtype, value.dtype, output.dtype, query.device,
               working_key.data_ptr(), working_value.data_ptr(), working_lens.data_ptr(), workspace.data_ptr(),
               slots.data_ptr(), slots.shape, slots.dtype, slots.device,
               None if positions is None else (positions.data_ptr(), positions.shape, positions.dtype,
                                               positions.device), float(scale))
    if sig is not None:
        args = reuse.get(sig)
        if args is not None:
            args[0] = _lib.stream_handle(query.device)
            args[2], args[5], args[8], args[11] = (query.data_ptr(), key.data_ptr(), value.data_ptr(),
                                                   output.data_ptr())
            _lib.check(_lib.load().ds_draft_attention(*args))
            return output
    num_slots, hkv, budget, head_dim = working_key.shape
    if working_value.shape != working_key.shape:
        raise ValueError("working key and value caches must have the same shape")
    if not (working_key.is_contiguous() and working_value.is_contiguous()):
        raise ValueError("working caches must be contiguous")
    q = query.view(query.shape[0], -1, head_dim) if query.dim() == 2 else query
    hq = q.shape[1]
    if hq % hkv:
        raise ValueError("query heads must be a multiple of KV heads")
    out = output.view(output.shape[0], hq, head_dim) if output.dim() == 2 else output
    if out.shape[1:] != q.shape[1:]:
        raise ValueError("output must match the query's heads and head_dim")
    if isinstance(slots, torch.Tensor):
        rows = slots.numel()
    else:
        slots = list(slots)
        rows = len(slots)
    if rows > out.shape[0] or rows > q.shape[0]:
        raise RuntimeError("DiffSpec draft tensors omit active request rows")
    if positions is not None and not isinstance(positions, torch.Tensor):
        positions = list(positions)
        if len(positions) != rows:
            raise ValueError("one local position per pending row is required")
        if positions and max(positions) >= budget:
            raise RuntimeError("DiffSpec working cache exhausted")
        if positions and min(positions) < 0:
            raise ValueError("local positions must be non-negative")
    k = _as_heads(key, rows, hkv, head_dim, "key")
    v = _as_heads(value, rows, hkv, head_dim, "value")
    if q.stride(2) != 1 or out.stride(2) != 1:
        raise ValueError("query and output must be contiguous in head_dim")
    for t in (q, k, v, out, working_value):
        if t.dtype != working_key.dtype:
            raise ValueError("query, key, value, output and working caches must share a dtype")
    if working_lens.dtype != torch.int32 or not working_lens.is_contiguous() or working_lens.numel() < num_slots:
        raise ValueError("working_lens must be a contiguous int32 tensor with one entry per slot")
    if workspace.dtype != torch.uint8 or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous uint8 tensor")
    device = _lib.require_gpu(q, k, v, out, working_key, working_value, working_lens, workspace)
    slot_t = _int32_rows(slots, rows, device, "slots")
    pos_t = None if positions is None else _int32_rows(positions, rows, device, "positions")
    args = [
        _lib.stream_handle(device), _lib.dtype_code(working_key.dtype),
        q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1),
        working_key.data_ptr(), working_value.data_ptr(), working_lens.data_ptr(),
        slot_t.data_ptr() if rows else None, _lib.ptr(pos_t) if rows else None,
        rows, out.shape[0], num_slots, hq, hkv, head_dim, budget, float(scale),
        workspace.data_ptr(), workspace.numel(),
    ]
    _lib.check(_lib.load().ds_draft_attention(*args))
    if (sig is not None and rows and slot_t.data_ptr() == slots.data_ptr()
            and (positions is None or pos_t.data_ptr() == positions.data_ptr())):
        # Same tensors next time: only the activations' addresses change.
        if len(reuse) >= 64:
            reuse.clear()
        reuse[sig] = args
    return output
