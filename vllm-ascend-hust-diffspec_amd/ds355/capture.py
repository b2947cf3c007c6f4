"""Raw pre-RoPE K/V capture of draft tokens and the graph-safe RoPE input (one HIP launch).

Mirror of DiffSpecDraftCache._write_raw (diffspec/runtime.py:1602-1618), the
local positions of capture_raw_kv (:1797-1877) and graph_safe_rope_positions
(:1767-1794).  The reference builds index tensors on the host every draft
step; here the token-to-slot map is a device int32 array and one launch
scatters the rows, fills the cache-owned RoPE input and clears the previous
call's stale tail.
"""

from __future__ import annotations

import torch

from . import _lib

__all__ = ["capture_raw_kv_rows"]


def _rows(t: torch.Tensor, heads: int, head_dim: int, name: str) -> torch.Tensor:
    if t.dim() == 2 and t.shape[1] == heads * head_dim:
        if t.stride(1) != 1:
            raise ValueError(f"{name} must be contiguous in head_dim")
        return t.as_strided((t.shape[0], heads, head_dim), (t.stride(0), head_dim, 1))
    if t.dim() != 3 or t.shape[1:] != (heads, head_dim) or t.stride(2) != 1:
        raise ValueError(f"{name} must be [tokens, {heads}, {head_dim}] or [tokens, {heads * head_dim}]")
    return t


def capture_raw_kv_rows(
    key: torch.Tensor,
    value: torch.Tensor,
    raw_key: torch.Tensor,
    raw_value: torch.Tensor,
    token_slots: torch.Tensor,
    absolute_positions: torch.Tensor,
    rope_buffer: torch.Tensor | None,
    *,
    tokens: int,
    working_lens: torch.Tensor | None = None,
    local_positions: torch.Tensor | None = None,
    prev_count: int = 0,
    status: torch.Tensor | None = None,
    reuse: dict | None = None,
    reuse_key=None,
) -> torch.Tensor | None:
    """Scatter the first ``tokens`` rows of ``key``/``value`` into the raw caches
    at ``[token_slots[t], absolute_positions[t]]`` and write the RoPE input.

    The RoPE input is ``rope_buffer[:count]`` (``count`` = number of absolute
    positions), viewed with their shape: each draft row's working length when
    ``working_lens`` is given (0 for rows past ``tokens``), else
    ``local_positions``, else the absolute positions.  ``rope_buffer[count:
    prev_count]`` is zeroed.  Returns the view.  With ``rope_buffer=None``
    only the rows are scattered (``populate_prefill``) and None is returned.
    ``reuse`` (a dict the caller keeps) holds validated launch arguments per
    layout: a later call whose tensors differ only in their addresses skips
    the checks.  ``reuse_key`` replaces the layout key computed here when the
    caller knows it: everything the call takes but the addresses of ``key``,
    ``value`` and ``absolute_positions`` must then be the same for one key.
    """
    sig = None
    if reuse is not None and reuse_key is not None:
        sig = reuse_key
    elif reuse is not None:
        sig = (key.shape, key.stride(), value.shape, value.stride(), key.dtype, value.dtype, key.device,
               absolute_positions.shape, absolute_positions.stride(), absolute_positions.dtype,
               raw_key.data_ptr(), raw_value.data_ptr(), token_slots.data_ptr(), token_slots.numel(),
               token_slots.dtype, None if rope_buffer is None else rope_buffer.data_ptr(), tokens,
               None if working_lens is None else working_lens.data_ptr(),
               None if local_positions is None else (local_positions.data_ptr(), local_positions.shape,
                                                    local_positions.dtype),
               prev_count, None if status is None else status.data_ptr())
    if sig is not None:
        hit = reuse.get(sig)
        if hit is not None:
            args, view = hit
            args[0] = _lib.stream_handle(key.device)
            args[2], args[5], args[8] = key.data_ptr(), value.data_ptr(), absolute_positions.data_ptr()
            _lib.check(_lib.load().ds_capture_raw_kv(*args))
            return view
    num_slots, max_model_len, heads, head_dim = raw_key.shape
    if raw_value.shape != raw_key.shape or not (raw_key.is_contiguous() and raw_value.is_contiguous()):
        raise ValueError("raw key/value must have matching contiguous 4-D shapes")
    count = absolute_positions.numel()
    positions = absolute_positions.reshape(-1)
    if not positions.is_contiguous():
        raise ValueError("absolute positions must be contiguous")
    if positions.dtype not in (torch.int32, torch.int64):
        raise ValueError("absolute positions must be int32 or int64")
    if rope_buffer is None:
        if prev_count or working_lens is not None or local_positions is not None:
            raise ValueError("local positions and a stale tail need a RoPE buffer")
        count = 0  # scatter only
    elif rope_buffer.dtype != positions.dtype or not rope_buffer.is_contiguous():
        raise ValueError("the RoPE buffer must be contiguous with the positions' dtype")
    elif max(count, prev_count) > rope_buffer.numel():
        raise RuntimeError("DiffSpec RoPE input exceeds its persistent buffer")
    if tokens < 0 or tokens > positions.numel():
        raise ValueError("captured tokens must be between zero and the number of positions")
    k = _rows(key, heads, head_dim, "key")
    v = _rows(value, heads, head_dim, "value")
    if k.shape[0] < tokens or v.shape[0] < tokens:
        raise RuntimeError("DiffSpec draft tensors omit active request rows")
    if k.dtype != raw_key.dtype or v.dtype != raw_key.dtype:
        raise ValueError("key, value and raw caches must share a dtype")
    if token_slots.dtype != torch.int32 or not token_slots.is_contiguous() or token_slots.numel() < tokens:
        raise ValueError("token_slots must be a contiguous int32 tensor with one slot per captured token")
    local = None
    if local_positions is not None:
        local = local_positions.reshape(-1)
        if local.dtype != positions.dtype or not local.is_contiguous() or local.numel() < count:
            raise ValueError("local positions must match the absolute positions' dtype and count")
    if working_lens is not None and (working_lens.dtype != torch.int32 or not working_lens.is_contiguous()):
        raise ValueError("working_lens must be a contiguous int32 tensor")
    device = _lib.require_gpu(k, v, raw_key, raw_value, token_slots, positions, rope_buffer, working_lens, local,
                              status)
    args = [
        _lib.stream_handle(device), _lib.dtype_code(raw_key.dtype),
        k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
        positions.data_ptr(), 1 if positions.dtype == torch.int64 else 0,
        token_slots.data_ptr(), tokens, raw_key.data_ptr(), raw_value.data_ptr(),
        num_slots, max_model_len, heads, head_dim,
        _lib.ptr(working_lens), _lib.ptr(local), _lib.ptr(rope_buffer), count, prev_count, _lib.ptr(status),
    ]
    _lib.check(_lib.load().ds_capture_raw_kv(*args))
    view = None if rope_buffer is None else rope_buffer[:count].view(absolute_positions.shape)
    if sig is not None and positions.data_ptr() == absolute_positions.data_ptr():
        if len(reuse) >= 64:
            reuse.clear()
        reuse[sig] = (args, view)
    return view
