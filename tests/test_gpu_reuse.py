"""GPU parity of the gather records: a rebuild that leaves out unchanged tasks.

The reference rebuilds every row's working cache from the raw cache at every
compact prefill (diffspec/runtime.py:1737-1765).  ds355 keeps per-task gather
records (include/ds355.h) and moves only what changed: after a retrieval
every row, between retrievals only the rolling tail.  Optionally the
retrieval call moves each row's history prefix itself, before the draft's
prefill (diffspec/proposer.py:211-220, then :256-307), and the compact
prefill after it the rest.  These tests run whole draft cycles through
``DiffSpecDraftCache`` and compare every cycle's working cache with the
oracle's full per-request rebuild (runtime.py:1683-1711) on the same raw
cache, bit for bit; draft steps are simulated by writing garbage past each
row's history, as the draft attention and the raw capture do.
"""

from types import SimpleNamespace

import pytest
import torch

from helpers import O, gen

pytestmark = pytest.mark.gpu

CHUNK, BUDGET, WINDOW, QLEN, HQ, HKV, D, BLOCK = 64, 2048, 256, 5, 32, 4, 128, 128


class _Rotary:
    rotary_dim = D
    is_neox_style = True

    def __init__(self, cos_sin):
        self.cos_sin_cache = cos_sin


def _cache(cuda, rows, lmax, interval, cos_sin, prefix_at_retrieval=False):
    from ds355 import runtime

    settings = runtime.DiffSpecSettings(chunk_size=CHUNK, token_budget=BUDGET, retrieval_interval=interval,
                                        max_tree_nodes=4, max_tree_depth=4, tree_threshold=0.7,
                                        adaptive_profile=False, recent_window=WINDOW)
    return runtime.DiffSpecDraftCache(settings, max_num_reqs=rows, max_model_len=lmax, num_kv_heads=HKV, head_dim=D,
                                      target_num_layers=2, dtype=torch.bfloat16, device=cuda,
                                      rotary_embedding=_Rotary(cos_sin.to(cuda)),
                                      prefix_at_retrieval=prefix_at_retrieval)


def _expected(raw_k, raw_v, slots, committed, selections, cos_sin, shape):
    budget = O.history_budget(BUDGET, 4, CHUNK)
    exp_k = torch.full(shape, float("nan"), dtype=torch.bfloat16)
    exp_v = exp_k.clone()
    roots = O.rebuild_working_cache_per_request(raw_k, raw_v, exp_k, exp_v, slots, committed, selections, cos_sin,
                                                chunk_size=CHUNK, budget=budget, rotary_dim=D, is_neox_style=True,
                                                recent_window=WINDOW)
    return exp_k, exp_v, roots


def _same_history(cache, exp_k, exp_v, slots, roots):
    got_k, got_v = cache.working_key.cpu(), cache.working_value.cpu()
    for slot, n in zip(slots, roots):
        for got, exp in ((got_k, exp_k), (got_v, exp_v)):
            a, b = got[slot, :, :n], exp[slot, :, :n]
            assert torch.equal(a.isnan(), b.isnan()), slot
            assert torch.equal(torch.nan_to_num(a), torch.nan_to_num(b)), slot


@pytest.mark.parametrize("rows,prefix", [(10, True), (4, True), (10, False)],
                         ids=["prefix-single-launch", "prefix-chain", "rebuild-at-prefill"])
def test_draft_cycles_match_full_rebuilds(cuda, rows, prefix):
    """Eight draft cycles, retrieval every second one, and a request replaced
    in a reused slot halfway: each cycle's working cache equals the oracle's
    full rebuild of every row, and between retrievals the prefix tasks are
    recorded as held.  With ``prefix`` the retrieval call moves each row's
    history prefix (as one launch with the scoring at 8+ rows)."""
    budget = O.history_budget(BUDGET, 4, CHUNK)
    g = gen(41 + rows)
    lmax = 9000
    committed = [int(x) for x in torch.randint(3000, 7000, (rows,), generator=g)]
    raw_k = torch.randn((rows, lmax, HKV, D), generator=g).to(torch.bfloat16)
    raw_v = torch.randn((rows, lmax, HKV, D), generator=g).to(torch.bfloat16)
    cos_sin = O.rope_cos_sin_cache(D, BUDGET)
    cache = _cache(cuda, rows, lmax, 2, cos_sin, prefix_at_retrieval=prefix)
    cache.raw_key.copy_(raw_k)
    cache.raw_value.copy_(raw_v)
    cache.working_key.fill_(float("nan"))
    cache.working_value.fill_(float("nan"))
    pages = (lmax + BLOCK - 1) // BLOCK
    key_cache = torch.randn((rows * pages, BLOCK, HKV, D), generator=g).to(torch.bfloat16).to(cuda)
    table = torch.randperm(rows * pages, generator=g).to(torch.int32).view(rows, pages).to(cuda)
    ids = [f"r{i}" for i in range(rows)]
    selections: dict[int, torch.Tensor] = {}
    retrievals = 0
    for cycle in range(8):
        if cycle == 4:
            # Request r1 leaves; a new one takes its slot with another history.
            slot = cache._request_slots["r1"]
            ids[1] = "r1-new"
            committed[1] = int(torch.randint(3000, 7000, (1,), generator=g))
            selections.pop(slot, None)
        tlens = [c - 1 + QLEN for c in committed]
        counts = [int(x) for x in torch.randint(1, QLEN + 1, (rows,), generator=g)]
        ends = [QLEN * (r + 1) for r in range(rows)]
        meta = SimpleNamespace(actual_seq_lengths_q=ends, seq_lens_list=tlens, block_tables=table, num_prefills=0)
        query = torch.randn((rows * QLEN, HQ, D), generator=g).to(torch.bfloat16).to(cuda)
        lse = torch.zeros((rows * QLEN, HQ), dtype=torch.float32, device=cuda)
        cache.begin_target_forward(ids)
        slots = list(cache._active_slots)
        cache.capture_target_attention(query, lse, key_cache, meta, D ** -0.5)
        cache.accept_target_queries(torch.tensor(counts, dtype=torch.int32, device=cuda), is_prefill=False)
        status = cache.retrieval_status()
        retrieved = status["retrieval_count"] > retrievals
        retrievals = status["retrieval_count"]
        new_committed = [tl - QLEN + c for tl, c in zip(tlens, counts)]
        if retrieved:
            # The selection the GPU stored (its bit-exactness is tested elsewhere).
            scores = cache.scores[:rows].cpu()
            for r, slot in enumerate(slots):
                n = new_committed[r]
                sel = O.select_context_chunks(scores[r, : (n + CHUNK - 1) // CHUNK].contiguous(), n, CHUNK, budget)
                assert cache.sel_ids[slot, : sel.chunk_indices.numel()].cpu().tolist() == sel.chunk_indices.tolist()
                selections[slot] = sel.token_indices
        # The draft's prefill rewrites every verifier token's raw rows.
        cache.begin_cycle(ids)
        positions = [tl - QLEN + j for tl in tlens for j in range(QLEN)]
        key = torch.randn((rows * QLEN, HKV * D), generator=g).to(torch.bfloat16)
        value = torch.randn((rows * QLEN, HKV, D), generator=g).to(torch.bfloat16)
        cache.populate_prefill(torch.tensor(positions, dtype=torch.int64, device=cuda), key.to(cuda), value.to(cuda),
                               meta)
        O.write_raw(raw_k, raw_v, [slots[r] for r in range(rows) for _ in range(QLEN)], positions, key, value)
        committed = new_committed
        cache.prepare_compact_prefill(meta, rows, committed_seq_lens=committed)
        torch.cuda.synchronize()
        assert torch.equal(cache.raw_key.cpu(), raw_k) and torch.equal(cache.raw_value.cpu(), raw_v)
        exp_k, exp_v, roots = _expected(raw_k, raw_v, slots, committed, selections, cos_sin,
                                        tuple(cache.working_key.shape))
        assert cache.working_lens[slots].cpu().tolist() == roots, cycle
        _same_history(cache, exp_k, exp_v, slots, roots)
        if selections and not retrieved:
            held = int((cache.gather_records[slots] != 0).sum())
            assert held > 0, "no prefix task recorded as held between retrievals"
        # Draft steps: new rows past each history in the working cache, and
        # draft tokens' raw rows past each root (the next prefill rewrites them).
        for r, slot in enumerate(slots):
            n = roots[r]
            junk = torch.randn((HKV, 4, D), generator=g).to(torch.bfloat16)
            cache.working_key[slot, :, n:n + 4] = junk.to(cuda)
            cache.working_value[slot, :, n:n + 4] = junk.to(cuda)
            c = committed[r]
            draft = torch.randn((4, HKV, D), generator=g).to(torch.bfloat16)
            raw_k[slot, c:c + 4] = draft
            raw_v[slot, c:c + 4] = draft
            cache.raw_key[slot, c:c + 4] = draft.to(cuda)
            cache.raw_value[slot, c:c + 4] = draft.to(cuda)
        cache.end_cycle()
    assert retrievals == 4


def test_matching_record_leaves_a_task_alone(cuda):
    """White-box check that a held task is not moved: the same compact prefill
    twice, with one prefix position of the working cache overwritten in
    between, keeps the overwrite; after the slot's generation changes (a new
    request in the slot) the next rebuild restores it."""
    rows, lmax = 3, 6000
    budget = O.history_budget(BUDGET, 4, CHUNK)
    g = gen(47)
    raw_k = torch.randn((rows, lmax, HKV, D), generator=g).to(torch.bfloat16)
    raw_v = torch.randn((rows, lmax, HKV, D), generator=g).to(torch.bfloat16)
    cos_sin = O.rope_cos_sin_cache(D, BUDGET)
    cache = _cache(cuda, rows, lmax, 1, cos_sin)
    cache.raw_key.copy_(raw_k)
    cache.raw_value.copy_(raw_v)
    cache.working_key.zero_()  # defined bytes past each history, compared below
    cache.working_value.zero_()
    committed = [5000, 4500, 5900]
    # Stored selections: 31 chunk ids per slot, the newest chunk last.
    for slot, n in enumerate(committed):
        newest = (n - 1) // CHUNK
        chosen = sorted(torch.randperm(newest, generator=g)[:30].tolist()) + [newest]
        cache.sel_ids[slot, :31] = torch.tensor(chosen, dtype=torch.int32, device=cuda)
        cache.sel_count[slot] = 31
    cache.set_active_requests(["a", "b", "c"])
    meta = SimpleNamespace(seq_lens_list=committed)
    cache.prepare_compact_prefill(meta, rows, committed_seq_lens=committed)
    first = cache.working_key.clone()
    cache.working_key[1, :, 8:16] = 7.0
    cache.prepare_compact_prefill(meta, rows, committed_seq_lens=committed)
    torch.cuda.synchronize()
    assert bool((cache.working_key[1, :, 8:16] == 7.0).all()), "a held prefix task was moved again"
    bits = lambda t: t.view(torch.int16)  # noqa: E731  (bitwise: NaN-safe)
    assert torch.equal(bits(cache.working_key[0]), bits(first[0]))
    assert torch.equal(bits(cache.working_key[2]), bits(first[2]))
    cache.set_active_requests(["a", "c"])       # b leaves: its slot's generation changes
    cache.set_active_requests(["a", "c", "b"])  # and b comes back into the freed slot
    slot = cache._request_slots["b"]
    newest = (committed[1] - 1) // CHUNK
    chosen = sorted(torch.randperm(newest, generator=g)[:30].tolist()) + [newest]
    cache.sel_ids[slot, :31] = torch.tensor(chosen, dtype=torch.int32, device=cuda)
    cache.sel_count[slot] = 31
    order = [committed[0], committed[2], committed[1]]
    cache.prepare_compact_prefill(SimpleNamespace(seq_lens_list=order), rows, committed_seq_lens=order)
    torch.cuda.synchronize()
    selections = {}
    for s, n in zip(cache._active_slots, order):
        ids = cache.sel_ids[s, :31].cpu().tolist()
        tokens = [t for c in ids for t in range(c * CHUNK, min((c + 1) * CHUNK, n))]
        selections[s] = torch.tensor(tokens, dtype=torch.int64)
    exp_k, exp_v, roots = _expected(raw_k, raw_v, list(cache._active_slots), order, selections, cos_sin,
                                    tuple(cache.working_key.shape))
    _same_history(cache, exp_k, exp_v, list(cache._active_slots), roots)
    assert roots[2] >= 16
