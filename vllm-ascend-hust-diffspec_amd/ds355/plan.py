"""Device-side history plans — replaces diffspec/runtime.py:1713-1757.

The reference builds each plan row on the host (``_history_plan_host``),
copying a slot's selected chunk starts back from the device when the
selection changed, then uploads the padded plan tensor.  ``build_history_plans``
computes the same rows on the device from the per-slot selection state in one
launch, with no host round trip.
"""

from __future__ import annotations

import torch

from . import _lib


def history_budget(token_budget: int, max_tree_depth: int, chunk_size: int) -> int:
    """``((token_budget - K - 1) // chunk) * chunk`` (diffspec/runtime.py:627-637)."""
    budget = (token_budget - max_tree_depth - 1) // chunk_size * chunk_size
    if budget <= 0:
        raise ValueError("DiffSpec token budget is too small for tree tokens")
    return budget


def plan_width(token_budget: int, chunk_size: int) -> int:
    """Plan row width ``5 + token_budget // chunk`` (compact_kv.py:217-218)."""
    return 5 + token_budget // chunk_size


def build_history_plans(
    sel_ids: torch.Tensor,
    sel_count: torch.Tensor,
    slots: torch.Tensor,
    committed_lens: torch.Tensor,
    *,
    chunk_size: int,
    history_budget: int,
    token_budget: int,
    recent_window: int | None = None,
    working_lens: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Plan rows ``[R, 5 + token_budget // chunk]`` int64.

    Row r: slot ``slots[r]`` (padding when outside ``[0, num_slots)``), history
    end ``committed_lens[r] - 1``, the slot's selection ``sel_ids[slot,
    :sel_count[slot]]`` (``sel_count < 0``: none).  ``recent_window=None`` is
    the reference's rolling tail of one chunk.
    """
    device = _lib.require_gpu(sel_ids, sel_count, slots, committed_lens, working_lens, out)
    for name, t in (("sel_ids", sel_ids), ("sel_count", sel_count), ("slots", slots),
                    ("committed_lens", committed_lens)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 tensor")
    if working_lens is not None and (working_lens.dtype != torch.int32 or not working_lens.is_contiguous()):
        raise ValueError("working_lens must be a contiguous int32 tensor")
    rows = slots.numel()
    if committed_lens.numel() != rows:
        raise ValueError("slots and committed_lens must have one entry per row")
    width = plan_width(token_budget, chunk_size)
    if out is None:
        out = torch.empty((rows, width), dtype=torch.int64, device=device)
    elif out.shape != (rows, width) or out.dtype != torch.int64 or not out.is_contiguous():
        raise ValueError("plan output must be a contiguous int64 [rows, 5 + token_budget // chunk] tensor")
    window = chunk_size if recent_window is None else recent_window
    lib = _lib.load()
    _lib.check(lib.ds_build_plan(
        _lib.stream_handle(device), sel_ids.data_ptr(), sel_ids.stride(0), sel_count.data_ptr(),
        sel_count.numel(), slots.data_ptr(), committed_lens.data_ptr(), rows, chunk_size, history_budget,
        window, out.data_ptr(), width, _lib.ptr(working_lens),
    ))
    return out
