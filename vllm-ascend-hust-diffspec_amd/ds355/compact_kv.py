"""Fused raw-KV gather and local-position RoPE — drop-in for ``diffspec.compact_kv``.

``rebuild_compact_kv_from_plan`` keeps the signature, plan format, in-place
contract and ``ValueError`` messages of diffspec/compact_kv.py:136-242; the
Triton kernel is replaced by the HIP kernel ``ds_rebuild_compact_kv`` (one
ragged launch over all plan rows).
"""

from __future__ import annotations

import torch

from . import _lib


def _validate_compact_inputs(
    raw_key: torch.Tensor,
    raw_value: torch.Tensor,
    working_key: torch.Tensor,
    working_value: torch.Tensor,
    plan: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    *,
    max_width: int,
    rotary_dim: int,
) -> None:
    """Same checks and messages as diffspec/compact_kv.py:136-181."""
    if raw_key.ndim != 4 or raw_key.shape != raw_value.shape:
        raise ValueError("raw key/value must have matching 4-D shapes")
    if working_key.ndim != 4 or working_key.shape != working_value.shape:
        raise ValueError("working key/value must have matching 4-D shapes")
    slots, max_model_len, heads, head_dim = raw_key.shape
    if (
        working_key.shape[0] != slots
        or working_key.shape[1] != heads
        or working_key.shape[3] != head_dim
    ):
        raise ValueError("working cache slot, head and head dimensions must match raw KV")
    if min(max_model_len, heads, head_dim) <= 0:
        raise ValueError("raw sequence, head and head dimensions must be positive")
    if plan.ndim != 2 or plan.dtype != torch.int64:
        raise ValueError("KV plan must be a contiguous 2-D int64 tensor")
    if plan.shape[0] > slots or not 0 <= max_width <= working_key.shape[2]:
        raise ValueError("KV plan exceeds the working cache batch or token capacity")
    if rotary_dim < 0 or rotary_dim > head_dim or rotary_dim % 2:
        raise ValueError("rotary_dim must be even and between zero and head_dim")
    if (
        cos_sin_cache.ndim != 2
        or cos_sin_cache.shape[0] < max_width
        or cos_sin_cache.shape[1] < rotary_dim
        or cos_sin_cache.stride(1) != 1
    ):
        raise ValueError("cos/sin cache must contain all local positions and rotary dimensions")
    caches = (raw_key, raw_value, working_key, working_value)
    if any(not cache.is_contiguous() for cache in (*caches, plan)):
        raise ValueError("raw KV, working KV and plan must be contiguous")
    if any(cache.dtype != raw_key.dtype for cache in caches):
        raise ValueError("all KV caches must have the same dtype")
    if raw_key.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("KV caches must use BF16, FP16 or FP32")
    if any(tensor.device != raw_key.device for tensor in (*caches, plan, cos_sin_cache)):
        raise ValueError("KV caches, plan and cos/sin cache must share a device")


def check_plan_preconditions(plan: torch.Tensor, *, num_slots: int, max_model_len: int, token_budget: int,
                             chunk_size: int, row_active: torch.Tensor | None = None) -> None:
    """Preconditions the reference states but does not check (diffspec/compact_kv.py:199-205).

    Every active row with a history has a slot in ``[0, num_slots)`` that no
    other such row uses, ``history_len <= token_budget``, and decodes to
    positions inside ``[0, max_model_len)``.  Duplicate slots would make two
    rows write the same working rows concurrently.  Reads the plan back
    (host synchronisation): a debugging aid, run when ``DS355_DEBUG_CHECKS``
    is set.
    """
    rows = plan.detach().to("cpu").tolist()
    active = None if row_active is None else row_active.detach().to("cpu").tolist()
    seen: dict[int, int] = {}
    for r, row in enumerate(rows):
        slot, length, tail_start, prefix_len, drop = row[:5]
        if length <= 0 or (active is not None and not active[r]):
            continue
        if not 0 <= slot < num_slots:
            raise ValueError(f"plan row {r}: slot {slot} outside [0, {num_slots})")
        if slot in seen:
            raise ValueError(f"plan rows {seen[slot]} and {r} share slot {slot}; slots must be distinct")
        seen[slot] = r
        if length > token_budget or not 0 <= prefix_len <= length or drop < 0:
            raise ValueError(f"plan row {r}: inconsistent lengths {row[1:5]}")
        chunks = row[5:]
        last = prefix_len + drop - 1
        if prefix_len and (last // chunk_size >= len(chunks)
                           or not all(0 <= c * chunk_size < max_model_len for c in chunks[: last // chunk_size + 1])):
            raise ValueError(f"plan row {r}: prefix chunks outside the raw cache")
        if tail_start < 0 or tail_start + length - prefix_len > max_model_len:
            raise ValueError(f"plan row {r}: tail outside the raw cache")


def rebuild_compact_kv_from_plan(
    raw_key: torch.Tensor,
    raw_value: torch.Tensor,
    working_key: torch.Tensor,
    working_value: torch.Tensor,
    plan: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    *,
    chunk_size: int,
    max_width: int,
    rotary_dim: int,
    is_neox_style: bool,
    row_active: torch.Tensor | None = None,
) -> None:
    """Rebuild compact KV from fixed-capacity per-request chunk plans.

    A plan row contains ``[slot, history_len, tail_start, prefix_len,
    prefix_drop, chunk_ids...]`` with chunk capacity ``working_budget //
    chunk_size``.  Slots must be distinct across rows.  Padding after each
    row's ``history_len`` stays untouched.  ``max_width`` only bounds the
    launch; no plan value is read back to the host.  ``row_active`` (int32
    ``[rows]``, not in the reference) leaves rows whose flag is 0 untouched.
    """
    _validate_compact_inputs(
        raw_key, raw_value, working_key, working_value, plan, cos_sin_cache,
        max_width=max_width, rotary_dim=rotary_dim,
    )
    if chunk_size <= 0 or plan.shape[1] != 5 + working_key.shape[2] // chunk_size:
        raise ValueError("plan width must be 5 + working_budget // chunk_size")
    if not plan.shape[0] or not max_width:
        return
    device = _lib.require_gpu(raw_key, raw_value, working_key, working_value, plan, cos_sin_cache, row_active)
    if cos_sin_cache.dtype != raw_key.dtype:
        raise ValueError("cos/sin cache must use the KV dtype")
    if row_active is not None:
        if row_active.dtype != torch.int32 or row_active.numel() != plan.shape[0]:
            raise ValueError("row_active must be an int32 tensor with one flag per plan row")
        row_active = row_active.contiguous()
    lib = _lib.load()
    slots, max_model_len, heads, head_dim = raw_key.shape
    if _lib.DEBUG_CHECKS:
        check_plan_preconditions(plan, num_slots=slots, max_model_len=max_model_len,
                                 token_budget=working_key.shape[2], chunk_size=chunk_size, row_active=row_active)
    _lib.check(lib.ds_rebuild_compact_kv(
        _lib.stream_handle(device), _lib.dtype_code(raw_key.dtype),
        raw_key.data_ptr(), raw_value.data_ptr(), working_key.data_ptr(), working_value.data_ptr(),
        plan.data_ptr(), plan.shape[0], plan.shape[1],
        cos_sin_cache.data_ptr(), cos_sin_cache.stride(0), cos_sin_cache.shape[0],
        slots, max_model_len, heads, head_dim, working_key.shape[2], chunk_size, rotary_dim,
        1 if is_neox_style else 0, max_width, _lib.ptr(row_active),
    ))
