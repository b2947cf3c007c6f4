"""GPU parity: batched chunk selection (ds_select_chunks) and device plans (ds_build_plan).

Selection is judged bit-exact on identical score inputs (the reference's own
device test, tests/test_retrieval_npu.py:16-29, does the same).  Plans must
equal the oracle's ``history_plan`` row for row, and decode to the oracle's
``history_indices`` (tests/test_runtime.py:637-690).
"""

import random

import pytest
import torch

from helpers import O, gen

pytestmark = pytest.mark.gpu


def _select_rows(scores_rows, lengths, chunk, budget, device):
    from ds355.selection import select_context_chunks_batched

    width = max([s.numel() for s in scores_rows] + [1])
    scores = torch.zeros((len(scores_rows), width), dtype=torch.float32)
    for r, s in enumerate(scores_rows):
        scores[r, : s.numel()] = s
    ids, counts = select_context_chunks_batched(
        scores.to(device), torch.tensor(lengths, dtype=torch.int32, device=device), chunk, budget)
    ids, counts = ids.cpu(), counts.cpu()
    return [ids[r, : int(counts[r])].tolist() for r in range(len(scores_rows))]


@pytest.mark.parametrize("length", [2051, 32768, 40959])
def test_device_selection_preserves_exact_chronological_indices(cuda, length):
    from ds355.selection import select_context_chunks

    torch.manual_seed(17)
    scores = torch.randn((length + 63) // 64)
    expected = O.select_context_chunks(scores, length, 64, 2048)
    actual = select_context_chunks(scores.to(cuda), length, 64, 2048)
    assert torch.equal(actual.chunk_indices.cpu(), expected.chunk_indices)
    assert torch.equal(actual.token_indices.cpu(), expected.token_indices)
    torch.testing.assert_close(actual.chunk_scores.cpu(), expected.chunk_scores)
    # On tie-free inputs the oracle equals the reference's torch.topk formulation (runtime.py:375-390).
    rank = scores.clone()
    rank[-1] = float("-inf")
    topk = torch.cat((rank.topk(2048 // 64 - 1).indices, torch.tensor([scores.numel() - 1]))).sort().values
    assert torch.equal(expected.chunk_indices, topk)


def test_batched_selection_with_ties_and_edges(cuda):
    g = gen(21)
    chunk, budget = 16, 512  # K = 32
    rows, lengths = [], []
    for trial in range(72):
        kind = trial % 6
        length = int(torch.randint(0, 20000, (1,), generator=g))
        c = (length + chunk - 1) // chunk
        if kind == 0:
            s = torch.rand(c, generator=g)
        elif kind == 1:  # heavy ties: few distinct values
            s = torch.randint(0, 4, (c,), generator=g).float()
        elif kind == 2:  # all equal
            s = torch.full((c,), 0.5)
        elif kind == 3:  # a narrow band with repeats: duplicates inside one small threshold bucket
            s = 1.0 + torch.randint(0, 300, (c,), generator=g).float() * 1e-4
        elif kind == 4:  # chunk scores of one magnitude, as softmax means are
            s = (1.0 + 0.3 * torch.randn(c, generator=g)).abs() * 3e-5
        else:  # signed values, +-0 and infinities
            s = torch.randn(c, generator=g)
            if c > 4:
                s[0], s[1], s[2], s[3] = -0.0, 0.0, float("inf"), float("-inf")
        rows.append(s)
        lengths.append(length)
    lengths[5], rows[5] = 0, torch.zeros(0)
    lengths[6], rows[6] = 100, torch.rand(7, generator=g)  # C <= K
    actual = _select_rows(rows, lengths, chunk, budget, cuda)
    for r, (s, n) in enumerate(zip(rows, lengths)):
        expected = O.select_context_chunks(s, n, chunk, budget).chunk_indices.tolist()
        assert actual[r] == expected, r


def test_selection_from_global_keys_beyond_lds(cuda):
    """More candidates than the LDS key buffer (12288) read keys from global memory."""
    g = gen(8)
    chunk, budget = 16, 2048
    lengths = [16 * 20000 - 5, 16 * 12289 + 1]
    rows = [torch.rand((n + chunk - 1) // chunk, generator=g) for n in lengths]
    rows[1] = torch.randint(0, 50, rows[1].shape, generator=g).float()
    actual = _select_rows(rows, lengths, chunk, budget, cuda)
    for r, (s, n) in enumerate(zip(rows, lengths)):
        assert actual[r] == O.select_context_chunks(s, n, chunk, budget).chunk_indices.tolist()


def test_reference_selection_kat(cuda):
    """tests/test_runtime.py:301-310."""
    from ds355.selection import select_context_chunks

    scores = torch.tensor([0.1, 0.9, 0.8, 0.7, 0.01], device=cuda)
    selection = select_context_chunks(scores, seq_len=18, chunk_size=4, token_budget=12)
    assert selection.chunk_indices.tolist() == [1, 2, 4]
    assert selection.token_indices.tolist() == [4, 5, 6, 7, 8, 9, 10, 11, 16, 17]


def _device_plans(selections, slots, ends, chunk, budget, token_budget, recent_window, device, num_slots):
    from ds355.plan import build_history_plans

    capacity = token_budget // chunk
    sel_ids = torch.zeros((num_slots, capacity), dtype=torch.int32)
    sel_count = torch.full((num_slots,), -1, dtype=torch.int32)
    for slot, chunks in selections.items():
        if chunks is None:
            continue
        sel_count[slot] = len(chunks)
        sel_ids[slot, : len(chunks)] = torch.tensor(chunks, dtype=torch.int32)
    working_lens = torch.full((num_slots,), -7, dtype=torch.int32, device=device)
    plan = build_history_plans(
        sel_ids.to(device), sel_count.to(device), torch.tensor(slots, dtype=torch.int32, device=device),
        torch.tensor([e + 1 for e in ends], dtype=torch.int32, device=device), chunk_size=chunk,
        history_budget=budget, token_budget=token_budget, recent_window=recent_window, working_lens=working_lens,
    )
    return plan.cpu(), working_lens.cpu()


@pytest.mark.parametrize("chunk_size", [2, 8, 64])
def test_device_plans_match_host_plans_across_updates(cuda, chunk_size):
    rng = random.Random(17)
    token_budget = chunk_size * 8
    for budget_chunks in range(1, 8):
        budget = chunk_size * budget_chunks
        selections, slots, ends = {}, [], []
        for trial in range(60):
            slot = trial
            retrieval_end = rng.randint(1, 3072)
            scores = torch.tensor([rng.random() for _ in range((retrieval_end + chunk_size - 1) // chunk_size)])
            sel = O.select_context_chunks(scores, retrieval_end, chunk_size, budget)
            kind = trial % 3
            selections[slot] = sel.chunk_indices.tolist() if kind == 0 else ([] if kind == 1 else None)
            slots.append(slot)
            ends.append(max(0, retrieval_end + rng.randint(-4 * chunk_size, 4 * chunk_size)))
        plan, lens = _device_plans(selections, slots, ends, chunk_size, budget, token_budget, None, cuda, 60)
        for r, (slot, end) in enumerate(zip(slots, ends)):
            expected = O.history_plan(slot, selections[slot], end, chunk_size, budget)
            row = plan[r].tolist()
            assert row[: len(expected)] == expected, (budget, r)
            assert all(v == 0 for v in row[len(expected):])
            assert int(lens[slot]) == expected[1]
            decoded = O.decode_plan(expected, chunk_size)
            assert decoded == sorted(set(decoded)) and all(0 <= t < end for t in decoded)


def test_device_plans_with_recent_window_and_padding(cuda):
    rng = random.Random(5)
    chunk, token_budget = 64, 2048
    budget = O.history_budget(token_budget, 4, chunk)
    selections, slots, ends = {}, [], []
    for slot in range(20):
        end = rng.randint(1, 40000)
        scores = torch.tensor([rng.random() for _ in range((end + 1 + chunk - 1) // chunk)])
        selections[slot] = O.select_context_chunks(scores, end + 1, chunk, budget).chunk_indices.tolist()
        slots.append(slot)
        ends.append(end)
    slots_with_padding = slots + [-1, 99]
    ends_with_padding = ends + [10, 10]
    for window in (64, 256, 512):
        plan, lens = _device_plans(selections, slots_with_padding, ends_with_padding, chunk, budget, token_budget,
                                   window, cuda, 20)
        for r, (slot, end) in enumerate(zip(slots, ends)):
            expected = O.history_plan(slot, selections[slot], end, chunk, budget, recent_window=window)
            assert plan[r].tolist()[: len(expected)] == expected
            decoded = O.decode_plan(expected, chunk)
            indices = O.history_indices(
                torch.tensor([c * chunk + i for c in selections[slot] for i in range(chunk)]), end, chunk, budget,
                recent_window=window)
            assert decoded == indices.tolist()
        assert plan[20].abs().sum() == 0 and plan[21].abs().sum() == 0


@pytest.mark.parametrize("chunk,budget", [(32, 2016), (64, 1984), (16, 512), (8, 1024)])
def test_long_rows_shortlist_selection(cuda, chunk, budget):
    """Long rows (513 to 4096 chunks) with few picks, as long contexts with
    small chunks give: random scores, scores on a coarse grid so the cut
    falls inside a run of ties, NaN and infinities among the top, a dozen
    levels only, softmax-like means of one magnitude, and a few outliers over
    a tiny floor.  Bit-exact against the oracle."""
    g = gen(chunk + budget)
    rows, lengths = [], []
    for trial in range(48):
        kind = trial % 6
        c = int(torch.randint(513, 4097, (1,), generator=g))
        length = c * chunk - int(torch.randint(0, chunk, (1,), generator=g))
        if kind == 0:
            s = torch.rand(c, generator=g) * 1e-4
        elif kind == 1:  # ties at the cut: 300 levels
            s = torch.randint(0, 300, (c,), generator=g).float() * 1e-6
        elif kind == 2:  # NaN and +-inf among the largest
            s = torch.randn(c, generator=g)
            idx = torch.randint(0, c - 1, (6,), generator=g)
            s[idx[0]], s[idx[1]], s[idx[2]] = float("nan"), float("inf"), float("nan")
            s[idx[3]], s[idx[4]], s[idx[5]] = float("-inf"), -0.0, 0.0
        elif kind == 3:  # 12 levels: the shortlist overflows, radix select
            s = torch.randint(0, 12, (c,), generator=g).float()
        elif kind == 4:  # one magnitude, as softmax chunk means are
            s = (1.0 + 0.3 * torch.randn(c, generator=g)).abs() * 2.4e-5
        else:  # a few large outliers, the rest tiny
            s = torch.rand(c, generator=g) * 1e-7
            s[torch.randint(0, c - 1, (budget // chunk // 2,), generator=g)] = 1.0
        rows.append(s)
        lengths.append(length)
    actual = _select_rows(rows, lengths, chunk, budget, cuda)
    for r, (s, n) in enumerate(zip(rows, lengths)):
        assert actual[r] == O.select_context_chunks(s, n, chunk, budget).chunk_indices.tolist(), r
