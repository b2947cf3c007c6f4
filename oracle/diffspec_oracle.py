"""CPU oracle for the DiffSpec draft-context retrieval path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or as the timed CPU baseline),
never as the thing that is measured or shipped.

It restates, in plain PyTorch on the CPU, the reference plugin's algorithm for
one retrieval step: chunk scores -> top-k chunk selection -> history plan ->
gather + local-position RoPE + working-cache write.  Every function cites the
reference file and lines it follows (paths are relative to the reference
repository root).

How each function is pinned (checked against something other than itself) is
listed in ``PINNING`` at the bottom of this file; ``tests/test_oracle.py``
carries those checks, and ``tests/golden/`` holds the fixtures they write.

Parity unpinned (no fixture or known-answer test of the reference covers it):
  * the reference's CPU rotate goes through vLLM's external
    ``RotaryEmbedding.forward_native`` (diffspec/runtime.py:1629-1647), which
    every reference CPU test replaces with an identity rotary; this oracle
    rotates by the textbook neox / GPT-J formula in fp32 instead, pinned by a
    float64 recomputation, not by vLLM's code;
  * softmax LSE values come from torch_npu's fused attention in the reference
    (ascend_patch.py:205-239); here LSE is an input, built by the closed form
    ``logsumexp`` as the reference's own device test does.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

__all__ = [
    "Selection",
    "history_budget",
    "chunk_attention_scores",
    "paged_chunk_attention_scores",
    "select_context_chunks",
    "history_indices",
    "history_plan",
    "decode_plan",
    "pad_plan",
    "rope_cos_sin_cache",
    "rotate_local_key",
    "rebuild_compact_kv_from_plan",
    "rebuild_working_cache_per_request",
    "retrieval_rows",
    "retrieval_step",
    "draft_linear_attention",
    "write_raw",
    "graph_safe_rope_positions",
    "to_bf16_rne",
]


@dataclass(frozen=True)
class Selection:
    """Mirror of ``DiffSpecSelection`` (diffspec/runtime.py:44-48)."""

    chunk_indices: torch.Tensor
    token_indices: torch.Tensor
    chunk_scores: torch.Tensor


def history_budget(token_budget: int, max_tree_depth: int, chunk_size: int) -> int:
    """Selection / history capacity (diffspec/runtime.py:627-637).

    ``((token_budget - K - 1) // chunk) * chunk``; the working cache still has
    ``token_budget`` rows, the remainder is room for the K draft tokens and the
    root.
    """
    budget = (token_budget - max_tree_depth - 1) // chunk_size * chunk_size
    if budget <= 0:
        raise ValueError("DiffSpec token budget is too small for tree tokens")
    return budget


def chunk_attention_scores(
    query: torch.Tensor,
    keys: torch.Tensor,
    chunk_size: int,
    softmax_lse: torch.Tensor | None = None,
    scale: float | None = None,
    head_reduce: str = "mean",
) -> torch.Tensor:
    """Dense per-chunk attention mass (diffspec/runtime.py:281-345).

    query ``[Hq, D]``, keys ``[L, Hkv, D]`` -> fp32 ``[ceil(L / chunk)]``.
    ``mean`` head reduction is the reference (``chunk_mass.mean(dim=0)``,
    runtime.py:345).  ``max`` is the optional variant: per token, the largest
    weight over query heads, then the mean over the chunk's tokens.
    """
    if query.ndim != 2 or keys.ndim != 3:
        raise ValueError("query must be 2-D and keys must be 3-D")
    num_query_heads, head_dim = query.shape
    num_tokens, num_kv_heads, key_head_dim = keys.shape
    if head_dim != key_head_dim:
        raise ValueError("query and key head dimensions must match")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("query heads must be divisible by KV heads")
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    if num_tokens == 0:
        return torch.empty(0, dtype=torch.float32)
    group = num_query_heads // num_kv_heads
    # runtime.py:313-319: grouped einsum over fp32 copies, then scale.
    grouped = query.float().reshape(num_kv_heads, group, head_dim)
    logits = torch.einsum("hgd,thd->hgt", grouped, keys.float())
    logits = logits.reshape(num_query_heads, num_tokens)
    logits.mul_(scale if scale is not None else 1.0 / math.sqrt(head_dim))
    # runtime.py:321-327: supplied LSE, or the exact one.
    if softmax_lse is None:
        softmax_lse = torch.logsumexp(logits, dim=-1)
    else:
        softmax_lse = softmax_lse.float().reshape(-1)
        if softmax_lse.numel() != num_query_heads:
            raise ValueError("softmax_lse must contain one value per query head")
    mass = torch.exp(logits - softmax_lse[:, None])
    num_chunks = (num_tokens + chunk_size - 1) // chunk_size
    padded = num_chunks * chunk_size
    valid = torch.full((num_chunks,), float(chunk_size), dtype=torch.float32)
    valid[-1] = num_tokens - (num_chunks - 1) * chunk_size
    if head_reduce == "max":
        per_token = mass.max(dim=0).values
        if padded != num_tokens:
            per_token = torch.nn.functional.pad(per_token, (0, padded - num_tokens))
        return per_token.reshape(num_chunks, chunk_size).sum(dim=-1).div_(valid)
    if head_reduce != "mean":
        raise ValueError("head_reduce must be 'mean' or 'max'")
    # runtime.py:329-345: pad to a chunk multiple, sum, mean over heads, divide.
    if padded != num_tokens:
        mass = torch.nn.functional.pad(mass, (0, padded - num_tokens))
    chunk_mass = mass.reshape(num_query_heads, num_chunks, chunk_size).sum(dim=-1)
    return chunk_mass.mean(dim=0).div_(valid)


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
    """Paged scores with the reference kernel's output contract.

    Follows diffspec/kernels.py:11-150: for each row ``b`` the keys of tokens
    ``t < seq_lens[b]`` are read through ``block_table[b, t // block_size]``;
    the output is ``[B, ceil(max_seq_len / chunk)]`` fp32 and chunks beyond a
    row's length are 0 (``valid_count = 0`` -> ``0 / max(0, 1)``,
    kernels.py:80-82).  The maths per row is ``chunk_attention_scores`` with
    the supplied LSE, or, for ``softmax_lse=None``, with each head's
    ``logsumexp`` over the row's own tokens (runtime.py:321-322).
    """
    batch, num_query_heads, head_dim = query.shape
    _, block_size, num_kv_heads, _ = key_cache.shape
    lse = None if softmax_lse is None else softmax_lse.float().reshape(batch, num_query_heads)
    max_chunks = (max_seq_len + chunk_size - 1) // chunk_size
    out = torch.zeros((batch, max_chunks), dtype=torch.float32)
    for b in range(batch):
        length = int(seq_lens[b])
        if length <= 0:
            continue
        pages = (length + block_size - 1) // block_size
        table = block_table[b, :pages].long()
        dense = key_cache[table].reshape(-1, num_kv_heads, head_dim)[:length]
        row = chunk_attention_scores(
            query[b], dense, chunk_size, softmax_lse=None if lse is None else lse[b], scale=scale,
            head_reduce=head_reduce,
        )
        out[b, : row.numel()] = row
    return out


def select_context_chunks(
    chunk_scores: torch.Tensor,
    seq_len: int,
    chunk_size: int,
    token_budget: int,
) -> Selection:
    """Top chunks plus the forced newest chunk (diffspec/runtime.py:348-414).

    ``token_budget`` here is the caller's history budget (runtime.py:1560-1565).
    Ranking: the newest chunk is excluded from the ranking (runtime.py:376-377
    sets it to -inf) and appended; the other ``max_chunks - 1`` are the highest
    scores.  Ties are broken deterministically by the lower chunk index (a
    stable descending sort); on tie-free inputs this equals ``torch.topk``
    (runtime.py:378).  The result is sorted ascending (runtime.py:385-390).
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
    if num_chunks == 0:
        empty = torch.empty(0, dtype=torch.long)
        return Selection(empty, empty, chunk_scores)
    max_chunks = token_budget // chunk_size
    if num_chunks <= max_chunks:
        selected = torch.arange(num_chunks, dtype=torch.long)
    else:
        newest = num_chunks - 1
        order = torch.sort(chunk_scores[:newest].float(), descending=True, stable=True).indices
        selected = torch.cat((order[: max_chunks - 1], torch.tensor([newest])))
        selected = selected.sort().values
    offsets = torch.arange(chunk_size, dtype=torch.long)
    if seq_len % chunk_size:
        full = (selected[:-1, None] * chunk_size + offsets[None, :]).reshape(-1)
        tail = torch.arange((num_chunks - 1) * chunk_size, seq_len, dtype=torch.long)
        tokens = torch.cat((full, tail))
    else:
        tokens = (selected[:, None] * chunk_size + offsets[None, :]).reshape(-1)
    return Selection(selected, tokens, chunk_scores.index_select(0, selected))


def _tail_length(history_end: int, chunk_size: int, budget: int, recent_window: int | None) -> int:
    window = chunk_size if recent_window is None else recent_window
    return min(history_end, window, budget)


def history_indices(
    selected_tokens: torch.Tensor | None,
    history_end: int,
    chunk_size: int,
    budget: int,
    recent_window: int | None = None,
) -> torch.Tensor:
    """Working-cache history tokens (diffspec/runtime.py:1650-1681).

    With a selection: the selected tokens before the rolling tail and before
    the newest selected chunk, keeping the last ``budget - tail`` of them,
    then the tail ``[tail_start, history_end)``.  Without one: the last
    ``budget`` tokens.  ``recent_window=None`` is the reference (tail of
    ``min(chunk, budget)`` tokens); other values only change the tail length.
    """
    if selected_tokens is not None:
        tail_len = _tail_length(history_end, chunk_size, budget, recent_window)
        tail_start = history_end - tail_len
        selected = selected_tokens.long()
        prefix = selected[(selected >= 0) & (selected < tail_start)]
        if selected.numel():
            newest_start = int(selected[-1]) // chunk_size * chunk_size
            prefix = prefix[prefix < newest_start]
        tail = torch.arange(tail_start, history_end, dtype=torch.long)
        prefix_budget = budget - tail.numel()
        prefix = prefix[-prefix_budget:] if prefix_budget else selected[:0]
        return torch.cat((prefix, tail))
    start = max(0, history_end - budget)
    return torch.arange(start, history_end, dtype=torch.long)


def history_plan(
    slot: int,
    selected_chunks: list[int] | None,
    history_end: int,
    chunk_size: int,
    budget: int,
    recent_window: int | None = None,
) -> list[int]:
    """Compact encoding of ``history_indices`` (diffspec/runtime.py:1713-1735).

    ``[slot, history_len, tail_start, prefix_len, prefix_drop, *chunk_ids]``.
    ``selected_chunks`` is the sorted chunk-id list of the slot's selection
    (``selected[::chunk] // chunk``, runtime.py:1724-1725), ``[]`` for an empty
    selection and ``None`` when the slot has none.
    """
    if selected_chunks is None:
        length = min(history_end, budget)
        return [slot, length, history_end - length, 0, 0]
    tail_len = _tail_length(history_end, chunk_size, budget, recent_window)
    tail_start = history_end - tail_len
    if not selected_chunks:
        return [slot, tail_len, tail_start, 0, 0]
    chunks = [int(c) for c in selected_chunks]
    prefix_end = min(tail_start, chunks[-1] * chunk_size)
    prefix_tokens = sum(
        max(0, min(chunk_size, prefix_end - c * chunk_size)) for c in chunks
    )
    prefix_len = min(prefix_tokens, budget - tail_len)
    return [slot, prefix_len + tail_len, tail_start, prefix_len,
            prefix_tokens - prefix_len, *chunks]


def pad_plan(plans: list[list[int]], token_budget: int, chunk_size: int) -> torch.Tensor:
    """Plan tensor ``[R, 5 + token_budget // chunk]`` int64 (runtime.py:1753-1757)."""
    width = 5 + token_budget // chunk_size
    return torch.tensor([p + [0] * (width - len(p)) for p in plans], dtype=torch.long).reshape(-1, width)


def decode_plan(plan: list[int], chunk_size: int) -> list[int]:
    """Absolute positions of a plan row (tests/test_runtime.py:31-38; compact_kv.py:40-52)."""
    _, length, tail_start, prefix_len, prefix_drop, *chunks = [int(x) for x in plan]
    prefix = [
        chunks[(p + prefix_drop) // chunk_size] * chunk_size + (p + prefix_drop) % chunk_size
        for p in range(prefix_len)
    ]
    return prefix + list(range(tail_start, tail_start + length - prefix_len))


def rope_cos_sin_cache(
    rotary_dim: int, max_position: int, base: float = 1.0e6, dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Textbook RoPE table (Su et al., RoFormer 2021), ``[max_position, rotary_dim]``.

    Row ``p`` is ``[cos(p * f_i), sin(p * f_i)]`` with ``f_i = base^(-2i/rot)``,
    computed in fp32 and cast to the KV dtype, as the reference feeds the
    kernel (runtime.py:1758, ``_match_cos_sin_cache_dtype``).
    """
    inv_freq = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
    t = torch.arange(max_position, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).to(dtype)


def rotate_local_key(
    keys: torch.Tensor, cos_sin: torch.Tensor, rotary_dim: int, is_neox_style: bool,
) -> torch.Tensor:
    """RoPE at local positions ``0..n-1`` (diffspec/compact_kv.py:57-108, 122-133).

    keys ``[n, H, D]``.  fp32 maths on the dtype's values: ``o1 = x1*c - x2*s``,
    ``o2 = x2*c + x1*s``, each product and the sum rounded in fp32 (no fused
    multiply-add), then one rounding to the KV dtype.  Dimensions at and above
    ``rotary_dim`` are copied.  Neox pairs ``(i, i + rot/2)``; GPT-J pairs
    ``(2i, 2i + 1)``.
    """
    n = keys.shape[0]
    out = keys.clone()
    if rotary_dim == 0 or n == 0:
        return out
    half = rotary_dim // 2
    table = cos_sin[:n]
    cos = table[:, :half].float()[:, None, :]
    sin = table[:, half:rotary_dim].float()[:, None, :]
    if is_neox_style:
        first = keys[..., :half].float()
        second = keys[..., half:rotary_dim].float()
    else:
        pairs = keys[..., :rotary_dim].float().reshape(*keys.shape[:-1], half, 2)
        first, second = pairs[..., 0], pairs[..., 1]
    a = first * cos
    b = second * sin
    c = second * cos
    d = first * sin
    rotated_first = a - b
    rotated_second = c + d
    if is_neox_style:
        out[..., :half] = rotated_first.to(keys.dtype)
        out[..., half:rotary_dim] = rotated_second.to(keys.dtype)
    else:
        out[..., :rotary_dim] = torch.stack((rotated_first, rotated_second), dim=-1).reshape(
            *keys.shape[:-1], rotary_dim
        ).to(keys.dtype)
    return out


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
    row_active: list[bool] | None = None,
) -> None:
    """In-place rebuild of the working cache (diffspec/compact_kv.py:8-133, 184-242).

    raw ``[S, Lmax, H, D]`` -> working ``[S, H, budget, D]``.  For each plan row:
    decode the absolute positions, gather K/V, rotate K at local positions and
    write ``working[slot, :, :history_len]``; positions at or beyond
    ``history_len`` stay untouched.  ``row_active`` (not in the reference)
    leaves rows that keep their previous contents out entirely.
    """
    if not plan.shape[0] or not max_width:
        return
    for r in range(plan.shape[0]):
        if row_active is not None and not row_active[r]:
            continue
        row = [int(x) for x in plan[r].tolist()]
        slot, length = row[0], row[1]
        if length <= 0:
            continue
        positions = torch.tensor(decode_plan(row, chunk_size), dtype=torch.long)
        keys = raw_key[slot].index_select(0, positions)
        values = raw_value[slot].index_select(0, positions)
        rotated = rotate_local_key(keys, cos_sin_cache, rotary_dim, is_neox_style)
        working_key[slot, :, :length] = rotated.transpose(0, 1)
        working_value[slot, :, :length] = values.transpose(0, 1)


def rebuild_working_cache_per_request(
    raw_key: torch.Tensor,
    raw_value: torch.Tensor,
    working_key: torch.Tensor,
    working_value: torch.Tensor,
    slots: list[int],
    seq_lens: list[int],
    selections: dict[int, torch.Tensor | None],
    cos_sin_cache: torch.Tensor,
    *,
    chunk_size: int,
    budget: int,
    rotary_dim: int,
    is_neox_style: bool,
    recent_window: int | None = None,
) -> list[int]:
    """Per-request CPU branch (diffspec/runtime.py:1683-1711) with a real rotate.

    ``history_end = seq_len - 1``; indices from ``history_indices``; returns the
    history lengths (the roots' local positions).
    """
    lengths = []
    for slot, seq_len in zip(slots, seq_lens):
        end = max(0, seq_len - 1)
        idx = history_indices(selections.get(slot), end, chunk_size, budget, recent_window)
        n = idx.numel()
        keys = raw_key[slot].index_select(0, idx)
        values = raw_value[slot].index_select(0, idx)
        rotated = rotate_local_key(keys, cos_sin_cache, rotary_dim, is_neox_style)
        working_key[slot, :, :n] = rotated.transpose(0, 1)
        working_value[slot, :, :n] = values.transpose(0, 1)
        lengths.append(n)
    return lengths


def retrieval_rows(
    counts: list[int], query_ends: list[int], target_seq_lens: list[int], batch_size: int,
) -> tuple[list[int], list[int], list[int]]:
    """Rows, committed query indices and scored lengths (diffspec/runtime.py:1211-1276).

    Linear (non-tree) verification.  Rows past ``batch_size`` are graph
    padding and never scored (runtime.py:1214-1223); rows with no committed
    token keep their previous selection (runtime.py:1254); the query is the
    last committed one, ``start + clamp(count - 1, 0, qlen - 1)``
    (runtime.py:1246-1247); the scored length drops the rejected suffix,
    ``target_len - qlen + clamp(count, 1, qlen)`` (runtime.py:1265-1271).
    """
    ends = list(query_ends[:batch_size])
    starts = [0, *ends[:-1]]
    lens = [e - s for s, e in zip(starts, ends)]
    rows, q_index, lengths = [], [], []
    for i in range(batch_size):
        c = int(counts[i])
        if c <= 0:
            continue
        rows.append(i)
        q_index.append(starts[i] + min(max(c - 1, 0), lens[i] - 1))
        lengths.append(target_seq_lens[i] - lens[i] + min(max(c, 1), lens[i]))
    return rows, q_index, lengths


def retrieval_step(
    query: torch.Tensor,
    lse: torch.Tensor | None,
    key_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: list[int],
    raw_key: torch.Tensor,
    raw_value: torch.Tensor,
    working_key: torch.Tensor,
    working_value: torch.Tensor,
    slots: list[int],
    history_ends: list[int],
    cos_sin_cache: torch.Tensor,
    *,
    chunk_size: int,
    budget: int,
    token_budget: int,
    scale: float,
    rotary_dim: int,
    is_neox_style: bool,
    recent_window: int | None = None,
    regather: list[bool] | None = None,
    scores_override: torch.Tensor | None = None,
) -> dict:
    """One retrieval step on the CPU: score -> select -> plan -> gather.

    The composition of runtime.py:1282-1308 (scores, per-row selection),
    runtime.py:1737-1757 (plans) and compact_kv.py (gather / RoPE / write),
    used as the CPU baseline.  ``scores_override`` feeds externally computed
    scores to the selection, so selection parity can be judged on identical
    score inputs.
    """
    max_len = max(seq_lens) if seq_lens else 0
    if scores_override is None:
        scores = paged_chunk_attention_scores(
            query, key_cache, lse, block_table, torch.tensor(seq_lens, dtype=torch.int32),
            chunk_size=chunk_size, max_seq_len=max_len, scale=scale,
        )
    else:
        scores = scores_override
    selections: list[list[int]] = []
    plans = []
    for r, (length, slot, end) in enumerate(zip(seq_lens, slots, history_ends)):
        c = (length + chunk_size - 1) // chunk_size
        sel = select_context_chunks(scores[r, :c].contiguous(), length, chunk_size, budget)
        chunks = sel.chunk_indices.tolist()
        selections.append(chunks)
        plans.append(history_plan(slot, chunks, end, chunk_size, budget, recent_window))
    plan = pad_plan(plans, token_budget, chunk_size)
    width = max((p[1] for p in plans), default=0)
    rebuild_compact_kv_from_plan(
        raw_key, raw_value, working_key, working_value, plan, cos_sin_cache,
        chunk_size=chunk_size, max_width=width, rotary_dim=rotary_dim,
        is_neox_style=is_neox_style, row_active=regather,
    )
    return {"scores": scores, "selections": selections, "plan": plan}


def draft_linear_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    output: torch.Tensor,
    working_key: torch.Tensor,
    working_value: torch.Tensor,
    working_lens: list[int] | torch.Tensor,
    slots: list[int],
    positions: list[int],
) -> torch.Tensor:
    """Linear draft attention over the working cache, in place.

    Follows ``DiffSpecDraftCache.forward_attention`` (diffspec/runtime.py:2024-2077):
    ``output`` is zeroed (rows past ``len(slots)`` stay zero, as graph padding
    does in the batched NPU path, runtime.py:2097 and 2133); for row ``r`` with
    slot ``s`` and local position ``p`` the new key/value row is written at
    ``working[s, :, p]``, the working length becomes ``p + 1``, and every query
    head ``h`` attends over positions ``0..p`` of KV head ``h // G`` (the
    reference's ``repeat_interleave`` over the query-head axis).  Scores,
    softmax and the weighted sum are fp32 with fp32 values, as the reference's
    device test computes its expectation (tests/test_linear_attention_batch_npu.py:131-137;
    the CPU loop itself only runs with fp32 caches, since ``einsum`` does not
    mix fp32 probabilities with bf16 values); the result is rounded once to the
    output dtype.
    """
    output.zero_()
    kv_heads, head_dim = working_key.shape[1], working_key.shape[3]
    group = query.shape[1] // kv_heads
    for r, (slot, pos) in enumerate(zip(slots, positions)):
        working_key[slot, :, pos] = key[r].reshape(kv_heads, head_dim)
        working_value[slot, :, pos] = value[r].reshape(kv_heads, head_dim)
        working_lens[slot] = pos + 1
        keys = working_key[slot, :, : pos + 1].float()      # [Hkv, n, D]
        values = working_value[slot, :, : pos + 1].float()
        q = query[r].float().reshape(kv_heads, group, head_dim)
        logits = torch.matmul(q, keys.transpose(1, 2)) * scale  # [Hkv, G, n]
        weights = torch.softmax(logits, dim=-1)
        out = torch.matmul(weights, values).reshape(kv_heads * group, head_dim)
        output[r] = out.reshape(output[r].shape).to(output.dtype)
    return output


def write_raw(
    raw_key: torch.Tensor,
    raw_value: torch.Tensor,
    slots: list[int],
    positions: list[int],
    key: torch.Tensor,
    value: torch.Tensor,
) -> None:
    """Token ``t`` of ``key``/``value`` goes to ``raw[slots[t], positions[t]]``
    (``DiffSpecDraftCache._write_raw``, diffspec/runtime.py:1602-1618), every KV
    head at once; the rows are copies."""
    heads, head_dim = raw_key.shape[2], raw_key.shape[3]
    for t, (slot, pos) in enumerate(zip(slots, positions)):
        raw_key[slot, pos] = key[t].reshape(heads, head_dim)
        raw_value[slot, pos] = value[t].reshape(heads, head_dim)


def graph_safe_rope_positions(
    buffer: torch.Tensor,
    written: int,
    absolute_positions: torch.Tensor,
    local_positions: torch.Tensor | None,
) -> tuple[torch.Tensor, int]:
    """The cache-owned RoPE input (diffspec/runtime.py:1767-1794).

    ``buffer[:count]`` receives the local positions (or the absolute ones when
    there are none) and ``buffer[count:written]``, the previous call's stale
    prefix, is zeroed.  Returns the view, shaped like the absolute positions,
    and the new written count.
    """
    count = absolute_positions.numel()
    if count > buffer.numel():
        raise RuntimeError("DiffSpec RoPE input exceeds its persistent buffer")
    if count < written:
        buffer[count:written] = 0
    view = buffer[:count].view_as(absolute_positions)
    view.copy_(absolute_positions if local_positions is None else local_positions)
    return view, count


def to_bf16_rne(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 with round-to-nearest-even, done on the bit pattern.

    Independent of ``Tensor.to(torch.bfloat16)`` so that the oracle's rounding
    can itself be checked (NaN maps to the quiet NaN 0x7fc0).
    """
    bits = x.float().contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    nan = torch.isnan(x.float())
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    rounded = torch.where(nan, torch.full_like(rounded, 0x7FC0), rounded) & 0xFFFF
    signed = torch.where(rounded >= 0x8000, rounded - 0x10000, rounded).to(torch.int16)
    return signed.view(torch.bfloat16)


# Which test pins which function, and against what.
PINNING = {
    "history_budget": "KAT values 1984/2016/3968 (runtime.py:627-635) and test_runtime.py settings",
    "chunk_attention_scores": "dense softmax formulation test_runtime.py:270-298; zero-K -> 1/L "
                              "(test_retrieval_dynamic_npu.py:39-42); planted missing partial-chunk divide",
    "paged_chunk_attention_scores": "dense GQA softmax reference with reordered pages "
                                    "(test_retrieval_npu.py:36-85), with a supplied LSE and without one "
                                    "(test_runtime.py:270-298); zero tail beyond a row",
    "select_context_chunks": "KATs test_runtime.py:301-310, 41-69, 532-605; brute force over subsets; "
                             "torch.topk on tie-free inputs",
    "history_indices": "KATs test_runtime.py:616-634, 781-799",
    "history_plan": "decode(plan) == history_indices, 200 randomised trials (test_runtime.py:637-690)",
    "decode_plan": "restated from test_runtime.py:31-38; checked by the KATs above",
    "rope_cos_sin_cache": "closed form at p=0 (cos 1, sin 0) and float64 recomputation",
    "rotate_local_key": "float64 complex multiplication within one bf16 rounding; identity at p=0; "
                        "GPT-J == neox under a dimension permutation",
    "rebuild_compact_kv_from_plan": "equals the per-request CPU branch (test_linear_attention_batch_npu.py:20-71); "
                                    "value KAT test_runtime.py:800-803",
    "retrieval_rows": "committed-query matrix test_runtime.py:72-142 and 532-605",
    "to_bf16_rne": "equals torch's fp32->bf16 cast on random and tie-heavy inputs",
    "retrieval_step": "composition of the pinned functions above; checked against them row by row",
    "write_raw": "value KAT of test_kv_graph_replay.py:59-73 (each step's row lands at its absolute position, "
                 "padding tokens are never written) and the exact-copy invariant on random rows",
    "graph_safe_rope_positions": "KATs test_kv_graph_replay.py:89-108 (dummy capture, replay, "
                                 "counts 8, 2, 7, 1, 0, 4 against a zero-tailed buffer)",
    "draft_linear_attention": "KAT of test_runtime.py:405-442 evaluated in closed form; single position -> "
                               "the new value row; zero query -> mean of values; GQA head map h // G (planted "
                               "h % Hkv map fails); NaN past each position never read "
                               "(test_linear_attention_batch_npu.py:109-112)",
}
