"""Shared input generators for the parity tests (seeded, CPU-side)."""

from __future__ import annotations

import math

import torch

from oracle import diffspec_oracle as O


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(shape, dtype, g) -> torch.Tensor:
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def rope_table_recipe(rotary_dim: int, rows: int = 128, dtype=torch.bfloat16) -> torch.Tensor:
    """cos/sin recipe of the reference's batched-rebuild device test
    (tests/test_linear_attention_batch_npu.py:32-33): phases = p * (1..rot/2) / 1000."""
    phases = torch.arange(rows, dtype=torch.float32)[:, None] * torch.arange(1, rotary_dim // 2 + 1)[None, :] / 1000
    return torch.cat((phases.cos(), phases.sin()), -1).to(dtype)


def paged_keys(lengths, num_kv_heads, head_dim, block_size, dtype, g, extra_blocks=3):
    """Paged K with a shuffled page order: returns (key_cache, block_table int32)."""
    pages = [(n + block_size - 1) // block_size for n in lengths]
    total = sum(pages) + extra_blocks
    key_cache = randn((total, block_size, num_kv_heads, head_dim), dtype, g)
    perm = torch.randperm(total, generator=g)
    width = max(max(pages), 1)
    table = torch.zeros((len(lengths), width), dtype=torch.int32)
    k = 0
    for b, p in enumerate(pages):
        table[b, :p] = perm[k:k + p].to(torch.int32)
        k += p
    return key_cache, table


def lse_for(query, key_cache, table, lengths, scale):
    """Exact per-head logsumexp over each row's keys, fp32 ``[B, Hq]``."""
    batch, hq, d = query.shape
    _, bs, hkv, _ = key_cache.shape
    out = torch.zeros((batch, hq), dtype=torch.float32)
    for b, n in enumerate(lengths):
        if n <= 0:
            continue
        pages = (n + bs - 1) // bs
        dense = key_cache[table[b, :pages].long()].reshape(-1, hkv, d)[:n].float()
        grouped = query[b].float().reshape(hkv, hq // hkv, d)
        logits = torch.einsum("hgd,thd->hgt", grouped, dense).reshape(hq, n) * scale
        out[b] = torch.logsumexp(logits, dim=-1)
    return out


def uniform_lengths(n, lo, hi, g):
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]


def max_ulp_bf16(a: torch.Tensor, b: torch.Tensor) -> int:
    """Largest distance in bf16 units in the last place (same-sign values)."""
    ai = a.contiguous().view(torch.int16).to(torch.int32)
    bi = b.contiguous().view(torch.int16).to(torch.int32)
    ai = torch.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = torch.where(bi < 0, -(bi & 0x7FFF), bi)
    return int((ai - bi).abs().max()) if a.numel() else 0


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


SCORE_RTOL = 1e-3  # chunk scores: within 1e-3 relative of the oracle, chunk by chunk
SCORE_FLOOR = 1e-12  # absolute slack for masses at the fp32 underflow edge (0.1% of a 1e-9 mass)


def assert_scores_close(actual: torch.Tensor, expected: torch.Tensor, rtol: float = SCORE_RTOL,
                        what: str = "scores") -> float:
    """Every chunk score within ``rtol`` of the oracle's, relative to that chunk's own value.

    ``|actual - expected| <= rtol * |expected| + 1e-12``: at 40k tokens a chunk
    holds about 2.5e-5 of the mass, so an absolute tolerance of the usual size
    would hide errors of several percent.  Zero chunks (beyond a row) must be
    zero.  Returns the largest relative error among chunks of mass >= 1e-9,
    which is printed.
    """
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, (a.shape, e.shape)
    err = (a - e).abs()
    bad = ~(err <= rtol * e.abs() + SCORE_FLOOR)  # NaN counts as bad
    mask = e.abs() >= 1e-9
    worst = float((err[mask] / e[mask].abs()).max()) if mask.any() else 0.0
    print(f"{what}: {int(mask.sum())} chunks, max relative error {worst:.3e}")
    if bad.any():
        i = int(bad.reshape(-1).nonzero()[0])
        raise AssertionError(f"{what}: {int(bad.sum())} chunks outside {rtol} relative; first at flat index {i}: "
                             f"{float(a.reshape(-1)[i])!r} vs {float(e.reshape(-1)[i])!r}")
    return worst


__all__ = ["O", "gen", "randn", "rope_table_recipe", "paged_keys", "lse_for", "uniform_lengths",
           "max_ulp_bf16", "default_scale", "assert_scores_close", "SCORE_RTOL"]


def attention_terms(q, work_k, work_v, slots, positions, scale) -> torch.Tensor:
    """sum_t softmax(scale q.k_t) |v_t| per (row, query head, d) in fp32, over positions 0..p
    of each row's slot in caches that already hold the new rows: the size of the terms a
    draft-attention output sums, which bounds its arithmetic error."""
    rows, hq, dim = q.shape
    group = hq // work_k.shape[1]
    out = torch.zeros((rows, hq, dim))
    for r, (slot, pos) in enumerate(zip(slots, positions)):
        k = work_k[slot, :, : pos + 1].float().repeat_interleave(group, dim=0)
        v = work_v[slot, :, : pos + 1].float().abs().repeat_interleave(group, dim=0)
        w = (torch.einsum("hd,hnd->hn", q[r].float(), k) * scale).softmax(-1)
        out[r] = torch.einsum("hn,hnd->hd", w, v)
    return out


def assert_attention_close(actual: torch.Tensor, expected: torch.Tensor, terms: torch.Tensor) -> None:
    """Each output within 2 ulps of its dtype of the oracle's fp32 result plus 2^-13 of its
    summed terms (``attention_terms``).

    The kernel multiplies V by the fp32 probabilities split into two 16-bit parts (within
    about 2^-15 of the fp32 product) and accumulates in fp32 in another order than the
    oracle, so an output that cancels to near zero carries the error of its terms.
    """
    rtol = 2 ** -7 if actual.dtype == torch.bfloat16 else 2 ** -10
    a, e = actual.float(), expected.float()
    assert torch.equal(a.isnan(), e.isnan())
    excess = (a - e).abs() - (rtol * e.abs() + 2 ** -13 * terms)
    worst = float(torch.nan_to_num(excess, nan=-1.0).max())
    err = float(torch.nan_to_num((a - e).abs(), nan=0.0).max())
    assert worst <= 0, f"output off by {worst:.3g} beyond the bound (max |error| {err:.3g})"
