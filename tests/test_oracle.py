"""Pins the CPU oracle against the reference's own known answers, closed forms,
brute force and invariants (CPU only).

Every oracle function is checked here against something other than itself;
the planted-mistake tests show that a plausible slip in the oracle (a missing
partial-chunk divide, a wrong tie order, a dropped tail) fails these checks.
"""

import itertools
import math
import random

import pytest
import torch

from helpers import rope_table_recipe
from oracle import diffspec_oracle as O


# -- history budget (runtime.py:627-637) --------------------------------------------------------
def test_history_budget_values():
    assert O.history_budget(2048, 4, 64) == 1984
    assert O.history_budget(2048, 4, 32) == 2016
    assert O.history_budget(4096, 4, 128) == 3968
    assert O.history_budget(8, 2, 2) == 4
    assert O.history_budget(128, 3, 32) == 96
    with pytest.raises(ValueError):
        O.history_budget(4, 4, 2)


# -- scores (runtime.py:281-345, kernels.py:11-150) ---------------------------------------------
def _dense_softmax_reference(query, keys, chunk, scale):
    """The reference test's independent formulation: softmax, then per-chunk means (test_runtime.py:278-287)."""
    hq = query.shape[0]
    expanded = keys.repeat_interleave(hq // keys.shape[1], dim=1)
    weights = (torch.einsum("hd,thd->ht", query.float(), expanded.float()) * scale).softmax(dim=-1)
    n = keys.shape[0]
    return torch.stack([weights[:, c:c + chunk].mean() for c in range(0, n, chunk)])


def test_dense_scores_match_reference_kat():
    torch.manual_seed(7)
    query = torch.randn(4, 8)
    keys = torch.randn(11, 2, 8)
    scale = 8 ** -0.5
    expected = _dense_softmax_reference(query, keys, 4, scale)
    torch.testing.assert_close(O.chunk_attention_scores(query, keys, 4, scale=scale), expected)
    expanded = keys.repeat_interleave(2, dim=1)
    lse = torch.logsumexp(torch.einsum("hd,thd->ht", query, expanded) * scale, dim=-1)
    torch.testing.assert_close(O.chunk_attention_scores(query, keys, 4, softmax_lse=lse, scale=scale), expected)


def test_planted_missing_partial_chunk_divide_is_caught():
    torch.manual_seed(7)
    query, keys, scale = torch.randn(4, 8), torch.randn(11, 2, 8), 8 ** -0.5
    good = O.chunk_attention_scores(query, keys, 4, scale=scale)
    planted = good.clone()
    planted[-1] = planted[-1] * 3 / 4  # divided by chunk (4) instead of the 3 valid tokens
    expected = _dense_softmax_reference(query, keys, 4, scale)
    assert not torch.allclose(planted, expected)


def test_zero_keys_give_one_over_length():
    for n in [1, 13, 100, 253]:
        q = torch.ones((4, 16))
        k = torch.zeros((n, 1, 16))
        lse = torch.full((4,), math.log(n))
        got = O.chunk_attention_scores(q, k, 16, softmax_lse=lse, scale=0.25)
        torch.testing.assert_close(got, torch.full_like(got, 1.0 / n))


@pytest.mark.parametrize("hq,hkv", [(4, 1), (8, 2), (6, 1), (12, 2)])
def test_paged_scores_equal_dense_with_reordered_pages(hq, hkv):
    torch.manual_seed(123)
    d, bs, chunk = 32, 16, 8
    lengths = [2 * bs + 13, bs + 5]
    query = torch.randn((2, hq, d), dtype=torch.bfloat16)
    keys = torch.randn((9, bs, hkv, d), dtype=torch.bfloat16)
    tables = torch.tensor([[4, 1, 7], [8, 2, 5]], dtype=torch.int32)
    scale = d ** -0.5
    lse, refs = [], []
    max_chunks = (max(lengths) + chunk - 1) // chunk
    for row, n in enumerate(lengths):
        dense = keys[tables[row].long()].reshape(-1, hkv, d)[:n]
        ref = torch.zeros(max_chunks)
        r = _dense_softmax_reference(query[row], dense, chunk, scale)
        ref[: r.numel()] = r
        refs.append(ref)
        expanded = dense.repeat_interleave(hq // hkv, dim=1)
        lse.append(torch.logsumexp(torch.einsum("hd,thd->ht", query[row].float(), expanded.float()) * scale, -1))
    got = O.paged_chunk_attention_scores(query, keys, torch.stack(lse), tables, torch.tensor(lengths),
                                         chunk_size=chunk, max_seq_len=max(lengths), scale=scale)
    torch.testing.assert_close(got, torch.stack(refs), rtol=1e-5, atol=1e-7)
    # Without an LSE each row normalises over its own tokens (runtime.py:321-322),
    # the softmax of the dense reference.
    free = O.paged_chunk_attention_scores(query, keys, None, tables, torch.tensor(lengths),
                                          chunk_size=chunk, max_seq_len=max(lengths), scale=scale)
    torch.testing.assert_close(free, torch.stack(refs), rtol=1e-5, atol=1e-7)
    # A planted LSE off by log 2 halves every score and is caught.
    off = O.paged_chunk_attention_scores(query, keys, torch.stack(lse) + math.log(2), tables, torch.tensor(lengths),
                                         chunk_size=chunk, max_seq_len=max(lengths), scale=scale)
    assert not torch.allclose(off, torch.stack(refs), rtol=1e-3)


def test_head_reduce_max_closed_form():
    torch.manual_seed(3)
    q, k = torch.randn(4, 8), torch.randn(10, 2, 8)
    got = O.chunk_attention_scores(q, k, 4, scale=0.3, head_reduce="max")
    w = (torch.einsum("hd,thd->ht", q, k.repeat_interleave(2, dim=1)) * 0.3).softmax(-1)
    per_token = w.max(dim=0).values
    expected = torch.stack([per_token[0:4].mean(), per_token[4:8].mean(), per_token[8:10].mean()])
    torch.testing.assert_close(got, expected)


# -- selection (runtime.py:348-414) -------------------------------------------------------------
def test_selection_reserves_partial_tail_kat():
    sel = O.select_context_chunks(torch.tensor([0.1, 0.9, 0.8, 0.7, 0.01]), 18, 4, 12)
    assert sel.chunk_indices.tolist() == [1, 2, 4]
    assert sel.token_indices.tolist() == [4, 5, 6, 7, 8, 9, 10, 11, 16, 17]


def test_tp_mean_selection_kat():
    """tests/test_runtime.py:41-69: mean of two ranks' scores selects tokens [2, 3, 6, 7, 8, 9]."""
    scores = (torch.tensor([0., 100., 0., 0., 0.]) + torch.tensor([0., 0., 0., 400., 0.])) / 2
    budget = O.history_budget(8, 1, 2)
    assert O.select_context_chunks(scores, 10, 2, budget).token_indices.tolist() == [2, 3, 6, 7, 8, 9]


def test_retrieval_kat_from_decode_cycle():
    """tests/test_runtime.py:578-600."""
    budget = O.history_budget(8, 2, 2)
    s = torch.tensor([[0.9, 0.1, 0.2], [0.1, 0.9, 0.0]])
    assert O.select_context_chunks(s[0, :3], 6, 2, budget).token_indices.tolist() == [0, 1, 4, 5]
    assert O.select_context_chunks(s[1, :2], 4, 2, budget).token_indices.tolist() == [0, 1, 2, 3]


def test_selection_equals_brute_force_on_tiny_inputs():
    rng = random.Random(1)
    for _ in range(300):
        chunk = rng.choice([1, 2, 3])
        k = rng.randint(1, 4)
        n = rng.randint(0, 9 * chunk)
        c = (n + chunk - 1) // chunk
        scores = torch.tensor(rng.sample(range(1000), c), dtype=torch.float32) / 7
        got = O.select_context_chunks(scores, n, chunk, k * chunk).chunk_indices.tolist()
        if c <= k:
            assert got == list(range(c))
            continue
        best = max(itertools.combinations(range(c - 1), k - 1), key=lambda s: sum(float(scores[i]) for i in s))
        assert got == sorted(list(best) + [c - 1])


def test_selection_equals_torch_topk_without_ties():
    g = torch.Generator().manual_seed(17)
    for n in [2051, 32768, 40959]:
        scores = torch.randn((n + 63) // 64, generator=g)
        rank = scores.clone()
        rank[-1] = float("-inf")
        topk = torch.cat((rank.topk(31).indices, torch.tensor([scores.numel() - 1]))).sort().values
        assert torch.equal(O.select_context_chunks(scores, n, 64, 2048).chunk_indices, topk)


def test_ties_prefer_lower_index_and_planted_order_is_caught():
    scores = torch.tensor([1.0, 2.0, 2.0, 2.0, 0.5, 9.0])
    got = O.select_context_chunks(scores, 6, 1, 3).chunk_indices.tolist()
    assert got == [1, 2, 5]
    planted = [2, 3, 5]  # higher index winning the tie
    assert got != planted


def test_special_values_rank_like_torch_sort():
    scores = torch.tensor([float("nan"), 1.0, -0.0, 0.0, float("inf"), float("-inf"), 3.0, 0.1])
    got = O.select_context_chunks(scores, 8, 1, 4).chunk_indices.tolist()
    assert got == [0, 4, 6, 7]  # NaN ranks highest, then +inf, then 3.0


# -- history / plan (runtime.py:1650-1735) ------------------------------------------------------
def test_history_rolls_tail_and_excludes_root():
    budget = O.history_budget(8, 2, 2)
    sel = torch.tensor([0, 1, 4, 5])
    assert O.history_indices(sel, 5, 2, budget).tolist() == [0, 1, 3, 4]
    assert O.history_indices(sel, 9, 2, budget).tolist() == [0, 1, 7, 8]


@pytest.mark.parametrize("selected,history_end,expected", [
    (list(range(65)), 64, list(range(64))),
    (list(range(70)), 64, list(range(64))),
    (list(range(32)) + list(range(96, 128)), 127, list(range(32)) + list(range(95, 127))),
    (list(range(12)), 11, list(range(11))),
])
def test_unique_committed_history_kat(selected, history_end, expected):
    budget = O.history_budget(128, 3, 32)
    assert O.history_indices(torch.tensor(selected), history_end, 32, budget).tolist() == expected


@pytest.mark.parametrize("history_end", [0, 5, 7, 9, 13, 15])
def test_plan_decodes_to_history(history_end):
    budget = O.history_budget(8, 2, 2)
    for selection in [None, [], [0, 1, 4, 5], [2, 3, 8, 9]]:
        tokens = None if selection is None else torch.tensor(selection, dtype=torch.long)
        chunks = None if selection is None else sorted({t // 2 for t in selection[::2]})
        expected = O.history_indices(tokens, history_end, 2, budget).tolist()
        assert O.decode_plan(O.history_plan(0, chunks, history_end, 2, budget), 2) == expected
        assert len(expected) <= budget and all(t < history_end for t in expected)


@pytest.mark.parametrize("chunk_size", [2, 8, 64])
@pytest.mark.parametrize("recent_window", [None, 1, 3, 100])
def test_plan_matches_history_randomised(chunk_size, recent_window):
    rng = random.Random(17)
    for _ in range(200):
        budget = chunk_size * rng.randint(1, 7)
        end_r = rng.randint(1, 3072)
        scores = torch.tensor([rng.random() for _ in range((end_r + chunk_size - 1) // chunk_size)])
        sel = O.select_context_chunks(scores, end_r, chunk_size, budget)
        end = max(0, end_r + rng.randint(-4 * chunk_size, 4 * chunk_size))
        for kind in ("retrieved", "empty", "none"):
            if kind == "retrieved":
                tokens, chunks = sel.token_indices, sel.chunk_indices.tolist()
            elif kind == "empty":
                tokens, chunks = torch.empty(0, dtype=torch.long), []
            else:
                tokens, chunks = None, None
            expected = O.history_indices(tokens, end, chunk_size, budget, recent_window).tolist()
            plan = O.history_plan(0, chunks, end, chunk_size, budget, recent_window)
            assert plan[1] == len(expected)
            assert O.decode_plan(plan, chunk_size) == expected
            assert len(expected) <= budget
            assert expected == sorted(set(expected))
            assert all(0 <= t < end for t in expected)


def test_planted_tail_mistake_is_caught():
    budget = O.history_budget(8, 2, 2)
    sel = torch.tensor([0, 1, 4, 5])
    planted = torch.cat((sel[sel < 4], torch.arange(4, 5)))  # tail that forgets to roll forward
    assert O.history_indices(sel, 9, 2, budget).tolist() != planted.tolist()


# -- RoPE (compact_kv.py:57-133) ----------------------------------------------------------------
def test_rope_table_closed_form():
    table = O.rope_cos_sin_cache(128, 64, dtype=torch.float32)
    assert torch.equal(table[0, :64], torch.ones(64)) and torch.equal(table[0, 64:], torch.zeros(64))
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    f = torch.arange(64, dtype=torch.float64)[:, None] * inv[None, :]
    # fp32 argument p * f_i is rounded before cos/sin: |error| <= p * 2^-24 + 1 ulp.
    torch.testing.assert_close(table.double(), torch.cat((f.cos(), f.sin()), -1), rtol=0, atol=1e-5)


@pytest.mark.parametrize("neox", [True, False])
def test_rotation_is_complex_multiplication(neox):
    g = torch.Generator().manual_seed(2)
    keys = torch.randn((50, 3, 64), generator=g).to(torch.bfloat16)
    table = rope_table_recipe(64, rows=50)
    out = O.rotate_local_key(keys, table, 64, neox)
    half = 32
    c = table[:, :half].double()[:, None, :]
    s = table[:, half:].double()[:, None, :]
    x = keys.double()
    if neox:
        z = torch.complex(x[..., :half], x[..., half:])
    else:
        z = torch.complex(x[..., 0::2], x[..., 1::2])
    r = z * torch.complex(c, s)
    exact = torch.cat((r.real, r.imag), -1) if neox else torch.stack((r.real, r.imag), -1).reshape(x.shape)
    # One rounding of an fp32 result: within one bf16 ulp of the exact product.
    ulp = torch.finfo(torch.bfloat16).eps * exact.abs().clamp_min(1e-30)
    assert ((out.double() - exact).abs() <= ulp + 1e-30).all()
    assert torch.equal(out[0], keys[0])  # position 0 is the identity


def test_gptj_equals_neox_under_dimension_permutation():
    g = torch.Generator().manual_seed(4)
    keys = torch.randn((20, 2, 16), generator=g).to(torch.bfloat16)
    table = rope_table_recipe(16, rows=20)
    perm = torch.cat((torch.arange(0, 16, 2), torch.arange(1, 16, 2)))
    neox = O.rotate_local_key(keys[..., perm], table, 16, True)
    gptj = O.rotate_local_key(keys, table, 16, False)
    assert torch.equal(neox, gptj[..., perm])


def test_partial_rotary_copies_the_tail():
    keys = torch.randn((10, 1, 32)).to(torch.bfloat16)
    out = O.rotate_local_key(keys, rope_table_recipe(16, rows=10), 16, True)
    assert torch.equal(out[..., 16:], keys[..., 16:])


def test_to_bf16_rne_matches_torch_cast():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(100000, generator=g) * torch.logspace(-30, 30, 100000)
    ties = (torch.arange(1, 2000, dtype=torch.int32) << 15 | 0x3F800000).view(torch.float32)
    for v in (x, ties, torch.tensor([0.0, -0.0, float("inf"), -float("inf")])):
        assert torch.equal(O.to_bf16_rne(v).view(torch.int16), v.to(torch.bfloat16).view(torch.int16))
    # NaN stays NaN (torch's vectorised cast uses another NaN payload than 0x7fc0).
    assert torch.isnan(O.to_bf16_rne(torch.tensor([float("nan")]))).all()


# -- rebuild (runtime.py:1683-1765, compact_kv.py) ----------------------------------------------
@pytest.mark.parametrize("heads,dim,rot,neox", [(2, 128, 128, True), (4, 256, 128, True), (2, 128, 64, False)])
@pytest.mark.parametrize("slots", [[0, 1], [2, 0]])
def test_plan_rebuild_equals_per_request_path(heads, dim, rot, neox, slots):
    g = torch.Generator().manual_seed(17)
    chunk, token_budget = 8, 64
    budget = O.history_budget(token_budget, 4, chunk)
    raw_k = torch.randn((3, 128, heads, dim), generator=g).to(torch.bfloat16)
    raw_v = torch.randn((3, 128, heads, dim), generator=g).to(torch.bfloat16)
    table = rope_table_recipe(rot)
    for end in [0, 1, 7, 62, 66, 73]:
        sels = {s: O.select_context_chunks(torch.arange((end + 7) // 8, dtype=torch.float32), end, chunk, budget)
                for s in slots}
        lengths = [end + 1, end + 6]
        a_k = torch.full((3, heads, token_budget, dim), float("nan"), dtype=torch.bfloat16)
        a_v, b_k, b_v = a_k.clone(), a_k.clone(), a_k.clone()
        n = O.rebuild_working_cache_per_request(raw_k, raw_v, a_k, a_v, slots, lengths,
                                                {s: v.token_indices for s, v in sels.items()}, table,
                                                chunk_size=chunk, budget=budget, rotary_dim=rot, is_neox_style=neox)
        plans = [O.history_plan(s, sels[s].chunk_indices.tolist(), max(0, L - 1), chunk, budget)
                 for s, L in zip(slots, lengths)]
        O.rebuild_compact_kv_from_plan(raw_k, raw_v, b_k, b_v, O.pad_plan(plans, token_budget, chunk), table,
                                       chunk_size=chunk, max_width=max(n), rotary_dim=rot, is_neox_style=neox)
        assert [p[1] for p in plans] == n
        assert torch.equal(torch.nan_to_num(a_k), torch.nan_to_num(b_k))
        assert torch.equal(torch.nan_to_num(a_v), torch.nan_to_num(b_v))
        for unused in set(range(3)) - set(slots):
            assert torch.isnan(b_k[unused]).all()


# -- verifier rows (runtime.py:1211-1276) -------------------------------------------------------
@pytest.mark.parametrize("counts", [[1, 2], [4, 4], [0, 2], [0, 0]])
@pytest.mark.parametrize("graph_padding", [False, True])
def test_committed_query_rows(counts, graph_padding):
    ends = [4, 8, 9] if graph_padding else [4, 8]
    seq_lens = [10, 12, 1] if graph_padding else [10, 12]
    rows, q_index, lengths = O.retrieval_rows(counts + ([3] if graph_padding else []), ends, seq_lens, 2)
    expected_rows = [i for i, c in enumerate(counts) if c > 0]
    assert rows == expected_rows
    assert q_index == [i * 4 + counts[i] - 1 for i in expected_rows]
    assert lengths == [seq_lens[i] - 4 + counts[i] for i in expected_rows]


# -- linear draft attention (runtime.py:2024-2077) ----------------------------------------------
def _attention_case(hkv, head_dim, budget, slots_total, dtype=torch.float32):
    work_k = torch.full((slots_total, hkv, budget, head_dim), float("nan"), dtype=dtype)
    return work_k, work_k.clone(), [0] * slots_total


def test_draft_attention_reference_kat():
    """The dense case of test_runtime.py:405-442 (one KV head, two query heads,
    positions 0..2), against its softmax evaluated in closed form."""
    work_k, work_v, lens = _attention_case(1, 2, 8, 1)
    work_k[0, 0, :2] = torch.tensor([[1.0, 0.0], [0.0, 1.0]])
    work_v[0, 0, :2] = torch.tensor([[2.0, 0.0], [0.0, 4.0]])
    query = torch.tensor([[[1.0, 1.0], [1.0, -1.0]]])
    out = torch.empty_like(query)
    O.draft_linear_attention(query, torch.tensor([[[1.0, 1.0]]]), torch.tensor([[[6.0, 8.0]]]), 2 ** -0.5, out,
                             work_k, work_v, lens, [0], [2])
    expected = torch.tensor([[[3.51744921742277, 5.020939060907324], [2.8559231488782837, 2.8320802581035918]]])
    torch.testing.assert_close(out, expected, rtol=1e-6, atol=1e-6)
    assert lens == [3]
    assert torch.equal(work_k[0, 0, 2], torch.tensor([1.0, 1.0]))
    assert torch.isnan(work_k[0, 0, 3:]).all()


def test_draft_attention_closed_forms():
    """Position 0 returns the new value row exactly; a zero query averages the
    values; rows past the batch are zero; NaN past each position is never read."""
    g = torch.Generator().manual_seed(5)
    hkv, d, budget = 2, 16, 32
    work_k, work_v, lens = _attention_case(hkv, d, budget, 3)
    work_k[1, :, :5] = torch.randn((hkv, 5, d), generator=g)
    work_v[1, :, :5] = torch.randn((hkv, 5, d), generator=g)
    query = torch.randn((4, 4 * hkv, d), generator=g)
    query[1] = 0.0
    key = torch.randn((4, hkv, d), generator=g)
    value = torch.randn((4, hkv, d), generator=g)
    out = torch.full_like(query, 7.0)
    O.draft_linear_attention(query, key, value, 0.25, out, work_k, work_v, lens, [2, 1], [0, 5])
    assert torch.equal(out[0], value[0].repeat_interleave(4, dim=0))
    mean = torch.cat([work_v[1, :, :5], value[1][:, None]], dim=1).mean(dim=1)
    torch.testing.assert_close(out[1], mean.repeat_interleave(4, dim=0), rtol=1e-6, atol=1e-6)
    assert not torch.isnan(out).any()
    assert out[2:].count_nonzero() == 0
    assert lens == [0, 6, 1]


def _planted_modulo_heads(query, key, value, scale, output, work_k, work_v, lens, slots, positions):
    """The oracle with a plausible slip: query head h reads KV head h % Hkv."""
    output.zero_()
    hkv = work_k.shape[1]
    for r, (slot, pos) in enumerate(zip(slots, positions)):
        work_k[slot, :, pos] = key[r]
        work_v[slot, :, pos] = value[r]
        lens[slot] = pos + 1
        heads = torch.arange(query.shape[1]) % hkv
        k = work_k[slot, heads, : pos + 1].float()
        v = work_v[slot, heads, : pos + 1].float()
        w = torch.softmax(torch.einsum("hd,hnd->hn", query[r].float(), k) * scale, dim=-1)
        output[r] = torch.einsum("hn,hnd->hd", w, v)
    return output


def test_draft_attention_group_map_is_repeat_interleave():
    """KV head j serves query heads j*G .. j*G+G-1: with constant values per KV
    head the output of head h is head h // G's value; the h % Hkv slip fails."""
    hkv, group, d = 2, 3, 8
    work_k, work_v, lens = _attention_case(hkv, d, 8, 1)
    work_k[0, :, :3] = 0.5
    work_v[0, 0, :3] = 1.0
    work_v[0, 1, :3] = 2.0
    query = torch.ones((1, hkv * group, d))
    key = torch.full((1, hkv, d), 0.5)
    value = torch.tensor([1.0, 2.0])[None, :, None].expand(1, hkv, d).clone()
    out = torch.empty_like(query)
    O.draft_linear_attention(query, key, value, 1.0, out, work_k.clone(), work_v.clone(), list(lens), [0], [3])
    assert torch.equal(out[0, :, 0], torch.tensor([1.0, 1.0, 1.0, 2.0, 2.0, 2.0]))
    slip = torch.empty_like(query)
    _planted_modulo_heads(query, key, value, 1.0, slip, work_k.clone(), work_v.clone(), list(lens), [0], [3])
    assert not torch.equal(slip[0, :, 0], out[0, :, 0])


def test_draft_attention_matches_float64_softmax():
    """Random GQA rows against a float64 softmax over the same prefix (bf16 output within one rounding)."""
    g = torch.Generator().manual_seed(9)
    hkv, group, d, budget = 2, 4, 32, 64
    work_k, work_v, lens = _attention_case(hkv, d, budget, 4, torch.bfloat16)
    positions, slots = [10, 0, 63], [3, 0, 2]
    for s, p in zip(slots, positions):
        work_k[s, :, :p] = torch.randn((hkv, p, d), generator=g).bfloat16()
        work_v[s, :, :p] = torch.randn((hkv, p, d), generator=g).bfloat16()
    query = torch.randn((3, hkv * group, d), generator=g).bfloat16()
    key = torch.randn((3, hkv, d), generator=g).bfloat16()
    value = torch.randn((3, hkv, d), generator=g).bfloat16()
    out = torch.empty_like(query)
    O.draft_linear_attention(query, key, value, d ** -0.5, out, work_k, work_v, lens, slots, positions)
    for r, (s, p) in enumerate(zip(slots, positions)):
        for h in range(hkv * group):
            k = work_k[s, h // group, : p + 1].double()
            v = work_v[s, h // group, : p + 1].double()
            logits = [float(query[r, h].double() @ k[t]) * d ** -0.5 for t in range(p + 1)]
            top = max(logits)
            w = torch.tensor([math.exp(x - top) for x in logits], dtype=torch.float64)
            ref = (w[:, None] * v).sum(0) / w.sum()
            torch.testing.assert_close(out[r, h].double(), ref, rtol=8e-3, atol=1e-5)


# -- raw KV capture and the RoPE input (runtime.py:1602-1618, 1767-1794) --------------------------
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_graph_safe_rope_positions_reference_kats(dtype):
    """tests/test_kv_graph_replay.py:89-108: one 12-entry buffer keeps its address, the
    replay's positions land first and every entry a previous call wrote beyond them is zero."""
    buffer = torch.zeros(12, dtype=dtype)
    captured, written = O.graph_safe_rope_positions(buffer, 0, torch.tensor([7, 8, 9, 10], dtype=dtype), None)
    assert captured.tolist() == [7, 8, 9, 10]
    replay, written = O.graph_safe_rope_positions(buffer, written, torch.tensor([7], dtype=dtype),
                                                  torch.tensor([4], dtype=dtype))
    assert replay.data_ptr() == captured.data_ptr()
    assert captured.tolist() == [4, 0, 0, 0]
    _, written = O.graph_safe_rope_positions(buffer, written, torch.tensor([7, 8, 9, 10], dtype=dtype),
                                             torch.tensor([5, 0, 0, 0], dtype=dtype))
    assert captured.tolist() == [5, 0, 0, 0]
    for count in [8, 2, 7, 1, 0, 4]:
        positions = torch.arange(count, dtype=dtype)
        _, written = O.graph_safe_rope_positions(buffer, written, positions, positions)
        expected = torch.zeros(12, dtype=dtype)
        expected[:count] = positions
        assert torch.equal(buffer, expected)
    with pytest.raises(RuntimeError, match="exceeds its persistent buffer"):
        O.graph_safe_rope_positions(buffer, written, torch.arange(13, dtype=dtype), None)


def test_write_raw_reference_kat():
    """tests/test_kv_graph_replay.py:59-73, 87: step s writes key (s+1, s+2), value +10 at
    absolute position 5+s of the one request; the padding tokens (position 11) are never written."""
    raw_k = torch.zeros((1, 12, 1, 2))
    raw_v = torch.zeros((1, 12, 1, 2))
    for step in range(3):
        key = torch.full((4, 2), 999.0)
        key[0] = torch.tensor([step + 1.0, step + 2.0])
        O.write_raw(raw_k, raw_v, [0], [5 + step], key[:1], key[:1] + 10)  # active rows only
        assert torch.equal(raw_k[0, 5 + step, 0], key[0])
        assert torch.equal(raw_v[0, 5 + step, 0], key[0] + 10)
    assert raw_k[0, 11].count_nonzero() == 0
    assert raw_k[0, :5].count_nonzero() == 0 and raw_k[0, 8:].count_nonzero() == 0
