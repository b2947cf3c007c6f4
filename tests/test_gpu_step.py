"""GPU parity: one retrieval step through ds_retrieval_step (score -> select -> plan -> gather).

Each case builds a verifier batch the way the plugin sees it (query tokens
per row, committed counts, graph-padding rows, paged target K, permuted
canonical slots) and checks every stage against the oracle:
  scores      within rtol 1e-3 (atol 1e-6);
  selection   bit-exact, judged on identical score inputs (the GPU's scores);
  plans       bit-exact;
  working KV  bit-exact (RoPE'd K within 1 bf16 ulp is the contract), and
              untouched (NaN) outside each row's history.
"""

import pytest
import torch

from helpers import O, assert_scores_close, default_scale, gen, max_ulp_bf16, paged_keys, randn

pytestmark = pytest.mark.gpu


def build_case(seed, *, real_rows, pad_rows, target_lens, query_len, counts, hq, hkv, head_dim, chunk,
               token_budget, block_size, lmax, slots, num_slots, depth=4, prev_counts=None, dtype=torch.bfloat16,
               neox=True):
    g = gen(seed)
    rows = real_rows + pad_rows
    qlens = [query_len] * real_rows + [1] * pad_rows
    tlens = list(target_lens) + [1] * pad_rows
    ends = [sum(qlens[: i + 1]) for i in range(rows)]
    starts = [0, *ends[:-1]]
    tokens = ends[-1]
    query = randn((tokens, hq, head_dim), dtype, g)
    lse = torch.randn((tokens, hq), generator=g)
    key_cache, table = paged_keys(tlens, hkv, head_dim, block_size, dtype, g)
    scale = default_scale(head_dim)
    # Exact LSE for each committed query over its causal prefix.
    _, q_index, lengths = O.retrieval_rows(counts, ends, tlens, real_rows)
    scored_rows = [i for i in range(real_rows) if counts[i] > 0]
    from helpers import lse_for
    exact = lse_for(query[q_index], key_cache, table[scored_rows], lengths, scale)
    for j, qi in enumerate(q_index):
        lse[qi] = exact[j]
    raw_k = randn((num_slots, lmax, hkv, head_dim), dtype, g)
    raw_v = randn((num_slots, lmax, hkv, head_dim), dtype, g)
    budget = O.history_budget(token_budget, depth, chunk)
    return dict(
        query=query, lse=lse, key_cache=key_cache, table=table, scale=scale, counts=counts + [0] * pad_rows,
        starts=starts, qlens=qlens, tlens=tlens, ends=ends, rows=rows, real_rows=real_rows,
        slots=slots + [-1] * pad_rows, num_slots=num_slots, raw_k=raw_k, raw_v=raw_v, chunk=chunk,
        token_budget=token_budget, budget=budget, hq=hq, hkv=hkv, head_dim=head_dim, lmax=lmax,
        committed=[tl - ql + min(max(c, 1), ql) for tl, ql, c in zip(tlens, qlens, counts + [0] * pad_rows)],
        cos_sin=O.rope_cos_sin_cache(head_dim, token_budget).to(dtype), dtype=dtype, neox=neox,
    )


@pytest.fixture(params=["chain", "fused"])
def path(request):
    """Both implementations of a full step: the three-kernel chain and the single launch."""
    return request.param


def run_gpu(case, device, *, stages=None, state=None, row_active=None, path="chain", single_launch=None,
            lse_free=False, flags=0, expect_status=0, recent_window=None, records=None, derive_committed=False):
    from ds355 import step

    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=device)  # noqa: E731
    rows = case["rows"]
    max_chunks = (max(case["tlens"]) + case["chunk"] - 1) // case["chunk"]
    if state is None:
        state = dict(
            scores=torch.zeros((rows, max_chunks), dtype=torch.float32, device=device),
            partials=torch.zeros((rows, max_chunks, case["hkv"]), dtype=torch.float32, device=device),
            sel_ids=torch.zeros((case["num_slots"], case["token_budget"] // case["chunk"]), dtype=torch.int32,
                                device=device),
            sel_count=torch.full((case["num_slots"],), -1, dtype=torch.int32, device=device),
            plan=torch.zeros((rows, 5 + case["token_budget"] // case["chunk"]), dtype=torch.int64, device=device),
            working_lens=torch.zeros((case["num_slots"],), dtype=torch.int32, device=device),
            work_k=torch.full((case["num_slots"], case["hkv"], case["token_budget"], case["head_dim"]),
                              float("nan"), dtype=case["dtype"], device=device),
            raw_k=case["raw_k"].to(device), raw_v=case["raw_v"].to(device),
            query=case["query"].to(device), lse=case["lse"].to(device), key_cache=case["key_cache"].to(device),
            table=case["table"].to(device), cos_sin=case["cos_sin"].to(device),
        )
        state["work_v"] = torch.full_like(state["work_k"], float("nan"))
    if lse_free and "lse_partials" not in state:
        state["lse_partials"] = torch.zeros((rows, max_chunks, case["hq"], 2), dtype=torch.float32, device=device)
        state["lse_out"] = torch.full((rows, case["hq"]), float("nan"), dtype=torch.float32, device=device)
    fused = path == "fused" and (stages is None or stages in (step.ALL, step.SCORE | step.SELECT | step.PREFIX))
    if fused and "workspace" not in state:
        state["workspace"] = step.new_workspace(rows, state["scores"].shape[1], case["hkv"], case["token_budget"],
                                                device)
    epoch = step.workspace_epoch(state["workspace"]) if fused else None
    step.retrieval_step(
        stages=step.ALL if stages is None else stages,
        snapshot=step.VerifierSnapshot(state["query"], None if lse_free else state["lse"], state["key_cache"],
                                       state["table"], case["scale"]),
        rows=step.VerifierRows(i32(case["counts"]), i32(case["starts"]), i32(case["qlens"]), i32(case["tlens"]),
                               case["real_rows"]),
        scores=state["scores"], score_partials=state["partials"], sel_ids=state["sel_ids"], sel_count=state["sel_count"], slots=i32(case["slots"]),
        committed_lens=None if derive_committed else i32(case["committed"]), plan=state["plan"],
        working_lens=state["working_lens"],
        raw_key=state["raw_k"], raw_value=state["raw_v"], working_key=state["work_k"],
        working_value=state["work_v"], cos_sin_cache=state["cos_sin"], rotary_dim=case["head_dim"],
        is_neox_style=case["neox"], chunk_size=case["chunk"], history_budget=case["budget"],
        recent_window=recent_window, row_active=None if row_active is None else i32(row_active),
        workspace=state.get("workspace") if fused else None,
        lse_partials=state.get("lse_partials") if lse_free else None,
        lse_out=state.get("lse_out") if lse_free else None, flags=flags, gather_records=records,
    )
    torch.cuda.synchronize()
    if fused:  # the single launch ran (epoch + 1) or, for other shapes, the chain did
        if single_launch is None:
            # Batches of fewer rows run the chain.
            single_launch = rows >= 8
        assert step.workspace_epoch(state["workspace"]) == epoch + (1 if single_launch else 0)
        if expect_status is not None:
            assert step.workspace_status(state["workspace"]) == expect_status
        assert step.workspace_launch_status(state["workspace"]) == 0  # handed over at the launch's end
    return state


def check_step(case, state, *, previous=None, row_active=None, recent_window=None):
    chunk, budget = case["chunk"], case["budget"]
    real = case["real_rows"]
    rows_idx, q_index, lengths = O.retrieval_rows(case["counts"], case["ends"], case["tlens"], real)
    gpu_scores = state["scores"].cpu()
    expected_scores = O.paged_chunk_attention_scores(
        case["query"][q_index], case["key_cache"], case["lse"][q_index], case["table"][rows_idx],
        torch.tensor(lengths), chunk_size=chunk, max_seq_len=max(lengths), scale=case["scale"])
    for j, b in enumerate(rows_idx):
        c = (lengths[j] + chunk - 1) // chunk
        assert_scores_close(gpu_scores[b, :c], expected_scores[j, :c])
    # Selection on identical (GPU) scores: bit-exact.
    selections = dict(previous or {})
    for j, b in enumerate(rows_idx):
        c = (lengths[j] + chunk - 1) // chunk
        sel = O.select_context_chunks(gpu_scores[b, :c].contiguous(), lengths[j], chunk, budget)
        selections[case["slots"][b]] = sel.chunk_indices.tolist()
    sel_count = state["sel_count"].cpu()
    sel_ids = state["sel_ids"].cpu()
    for slot, chunks in selections.items():
        assert int(sel_count[slot]) == len(chunks), slot
        assert sel_ids[slot, : len(chunks)].tolist() == chunks, slot
    # Plans, bit-exact; padding rows are all zero.
    plans = []
    for b in range(case["rows"]):
        slot = case["slots"][b]
        if slot < 0:
            assert state["plan"][b].abs().sum().item() == 0
            plans.append([0, 0, 0, 0, 0])
            continue
        plans.append(O.history_plan(slot, selections.get(slot), max(0, case["committed"][b] - 1), chunk, budget,
                                    recent_window))
    expected_plan = O.pad_plan(plans, case["token_budget"], chunk)
    assert torch.equal(state["plan"].cpu(), expected_plan)
    # Working cache.
    exp_k = torch.full(tuple(state["work_k"].shape), float("nan"), dtype=case["dtype"])
    exp_v = exp_k.clone()
    width = max(p[1] for p in plans)
    O.rebuild_compact_kv_from_plan(case["raw_k"], case["raw_v"], exp_k, exp_v, expected_plan, case["cos_sin"],
                                   chunk_size=chunk, max_width=width, rotary_dim=case["head_dim"],
                                   is_neox_style=case["neox"], row_active=row_active)
    got_k, got_v = state["work_k"].cpu(), state["work_v"].cpu()
    assert torch.equal(got_k.isnan(), exp_k.isnan())
    assert torch.equal(torch.nan_to_num(got_v), torch.nan_to_num(exp_v))
    assert max_ulp_bf16(torch.nan_to_num(got_k), torch.nan_to_num(exp_k)) <= 1
    assert torch.equal(torch.nan_to_num(got_k), torch.nan_to_num(exp_k))
    return selections


def test_single_request_8k(cuda, path):
    """One request, 8192 tokens, chunk 64, budget 2048 (K = 4 gives 1984 history tokens)."""
    case = build_case(0, real_rows=1, pad_rows=0, target_lens=[8192], query_len=1, counts=[1], hq=32, hkv=4,
                      head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=8192, slots=[0], num_slots=1)
    state = run_gpu(case, cuda, path=path)
    check_step(case, state)


def test_ragged_16_requests_40k(cuda, path):
    """16 requests, L ~ U[4096, 40960], contiguous slots in request order."""
    g = gen(1)
    lens = [int(x) for x in torch.randint(4096, 40961, (16,), generator=g)]
    case = build_case(1, real_rows=16, pad_rows=0, target_lens=lens, query_len=1, counts=[1] * 16, hq=32, hkv=4,
                      head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=40960,
                      slots=list(range(16)), num_slots=16)
    state = run_gpu(case, cuda, path=path)
    check_step(case, state)


def test_spec_decode_mask_padding_and_permuted_slots(cuda, path):
    """Batch 16 + 16 graph-padding rows, K = 4 draft tail with accepted 0..4, random slot permutation."""
    g = gen(4)
    lens = [int(x) for x in torch.randint(8192, 40961, (16,), generator=g)]
    accepted = [int(x) for x in torch.randint(0, 5, (16,), generator=g)]
    counts = [a + 1 for a in accepted]
    slots = [int(x) for x in torch.randperm(16, generator=g)]
    case = build_case(4, real_rows=16, pad_rows=16, target_lens=lens, query_len=5, counts=counts, hq=32, hkv=4,
                      head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=40960, slots=slots,
                      num_slots=16)
    state = run_gpu(case, cuda, path=path)
    check_step(case, state)


def test_zero_count_rows_keep_previous_selection(cuda, path):
    """Rows that committed nothing are not scored and keep their last selection (runtime.py:1254)."""
    g = gen(6)
    lens = [int(x) for x in torch.randint(3000, 9000, (6,), generator=g)]
    case = build_case(6, real_rows=6, pad_rows=2, target_lens=lens, query_len=5, counts=[1, 2, 3, 4, 5, 1],
                      hq=16, hkv=2, head_dim=64, chunk=32, token_budget=1024, block_size=64, lmax=9000,
                      slots=[5, 3, 1, 0, 2, 4], num_slots=6)
    state = run_gpu(case, cuda, path=path)
    first = check_step(case, state)
    # Next cycle: rows 1 and 4 commit nothing; the others advance by their count.
    case2 = dict(case)
    case2["counts"] = [2, 0, 1, 3, 0, 5, 0, 0]
    case2["committed"] = [tl - ql + min(max(c, 1), ql) for tl, ql, c in
                          zip(case["tlens"], case["qlens"], case2["counts"])]
    state["work_k"].fill_(float("nan"))  # fresh sentinel: only this cycle's writes are checked
    state["work_v"].fill_(float("nan"))
    state = run_gpu(case2, cuda, state=state, path=path)
    check_step(case2, state, previous=first)


def test_stress_64_rows_reuse_half(cuda, path):
    """64 rows, 8 KV heads / 64 q heads, chunk 128, budget 4096; half the rows keep their working rows."""
    g = gen(5)
    lens = [int(x) for x in torch.randint(2048, 6145, (64,), generator=g)]
    case = build_case(5, real_rows=64, pad_rows=0, target_lens=lens, query_len=1, counts=[1] * 64, hq=64, hkv=8,
                      head_dim=128, chunk=128, token_budget=4096, block_size=256, lmax=6144,
                      slots=list(range(64)), num_slots=64)
    state = run_gpu(case, cuda, path=path)
    check_step(case, state)
    full_k, full_v = state["work_k"].clone(), state["work_v"].clone()
    # Same step again with a random half flagged for reuse: the result must not change.
    active = [int(x) for x in (torch.rand(64, generator=g) < 0.5)]
    run_gpu(case, cuda, state=state, row_active=active, path=path)
    assert torch.equal(torch.nan_to_num(state["work_k"]), torch.nan_to_num(full_k))
    assert torch.equal(torch.nan_to_num(state["work_v"]), torch.nan_to_num(full_v))
    # Re-gathered rows really are rewritten; reused rows are not touched.
    state["work_k"].fill_(float("nan"))
    state["work_v"].fill_(float("nan"))
    run_gpu(case, cuda, state=state, row_active=active, path=path)
    for b in range(64):
        n = int(state["plan"][b, 1])
        if active[b]:
            assert torch.equal(state["work_k"][b, :, :n], full_k[b, :, :n])
        else:
            assert torch.isnan(state["work_k"][b]).all()


def test_stage_split_equals_full_chain(cuda, path):
    """SCORE | SELECT then PLAN (the runtime's two call sites) equals the one-call step."""
    from ds355 import step

    g = gen(7)
    lens = [int(x) for x in torch.randint(1000, 20000, (8,), generator=g)]
    case = build_case(7, real_rows=8, pad_rows=0, target_lens=lens, query_len=5, counts=[5, 1, 2, 3, 4, 5, 1, 2],
                      hq=32, hkv=4, head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=20000,
                      slots=[7, 6, 5, 4, 3, 2, 1, 0], num_slots=8)
    full = run_gpu(case, cuda, path=path)
    split = run_gpu(case, cuda, stages=step.SCORE | step.SELECT)
    assert torch.isnan(split["work_k"]).all()
    run_gpu(case, cuda, stages=step.PLAN, state=split)
    for key in ("scores", "sel_ids", "sel_count", "plan", "working_lens", "work_k", "work_v"):
        assert torch.equal(torch.nan_to_num(split[key]), torch.nan_to_num(full[key])), key


@pytest.mark.parametrize("seed,hq,hkv,head_dim,chunk,block_size", [(4, 32, 4, 128, 64, 128), (6, 16, 2, 64, 32, 64),
                                                                   (7, 12, 2, 64, 64, 128), (8, 64, 8, 64, 128, 128)])
def test_lse_free_step_equals_supplied_lse(cuda, path, seed, hq, hkv, head_dim, chunk, block_size):
    """Without a snapshot LSE the step computes each committed query's LSE over its
    scored tokens: the same normaliser the verifier's attention returns, so
    scores, selection, plans and working cache match the oracle with the exact
    LSE, and lse_out equals that LSE (groups of 8, 8, 6 and 8 query heads; 64 heads
    over 8 KV heads in the last case)."""
    g = gen(seed)
    lens = [int(x) for x in torch.randint(3000, 30000, (12,), generator=g)]
    counts = [int(x) for x in torch.randint(0, 6, (12,), generator=g)]
    counts[0] = 5
    slots = [int(x) for x in torch.randperm(12, generator=g)]
    case = build_case(seed, real_rows=12, pad_rows=4, target_lens=lens, query_len=5, counts=counts, hq=hq, hkv=hkv,
                      head_dim=head_dim, chunk=chunk, token_budget=2048, block_size=block_size, lmax=30000,
                      slots=slots, num_slots=12)
    state = run_gpu(case, cuda, path=path, lse_free=True)
    check_step(case, state)
    rows_idx, q_index, _ = O.retrieval_rows(case["counts"], case["ends"], case["tlens"], case["real_rows"])
    lse_out = state["lse_out"].cpu()
    torch.testing.assert_close(lse_out[rows_idx], case["lse"][q_index], rtol=1e-5, atol=1e-4)
    unscored = [b for b in range(case["rows"]) if b not in rows_idx]
    assert torch.isnan(lse_out[unscored]).all()  # rows that are not scored are left alone


@pytest.mark.parametrize("lse_free", [False, True])
def test_runtime_retrieval_and_rebuild_match_oracle(cuda, lse_free):
    """DiffSpecDraftCache end to end: verifier snapshot -> accept_target_queries (score +
    select) -> prepare_compact_prefill (plan + gather), against the oracle's step.  With
    lse_free_scoring the snapshot carries no LSE."""
    from types import SimpleNamespace

    from ds355 import runtime

    g = gen(21)
    lens = [int(x) for x in torch.randint(3000, 20000, (12,), generator=g)]
    counts = [int(x) for x in torch.randint(0, 6, (12,), generator=g)]
    counts[0] = 3
    case = build_case(21, real_rows=12, pad_rows=0, target_lens=lens, query_len=5, counts=counts, hq=32, hkv=4,
                      head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=20000,
                      slots=list(range(12)), num_slots=12)

    class Rotary:
        rotary_dim = 128
        is_neox_style = True
        cos_sin_cache = case["cos_sin"].to(cuda)

    settings = runtime.DiffSpecSettings(chunk_size=64, token_budget=2048, retrieval_interval=1, max_tree_nodes=4,
                                        max_tree_depth=4, tree_threshold=0.7, adaptive_profile=False)
    cache = runtime.DiffSpecDraftCache(settings, max_num_reqs=12, max_model_len=20000, num_kv_heads=4, head_dim=128,
                                       target_num_layers=2, dtype=torch.bfloat16, device=cuda,
                                       rotary_embedding=Rotary(), lse_free_scoring=lse_free)
    cache.raw_key.copy_(case["raw_k"])
    cache.raw_value.copy_(case["raw_v"])
    cache.working_key.fill_(float("nan"))
    cache.working_value.fill_(float("nan"))
    ids = [f"request-{i}" for i in range(12)]
    meta = SimpleNamespace(actual_seq_lengths_q=case["ends"], seq_lens_list=case["tlens"],
                           block_tables=case["table"].to(cuda), num_prefills=0)
    cache.begin_target_forward(ids)
    assert cache._active_slots == list(range(12))
    cache.capture_target_attention(case["query"].to(cuda), None if lse_free else case["lse"].to(cuda),
                                   case["key_cache"].to(cuda), meta, case["scale"])
    cache.accept_target_queries(torch.tensor(counts, dtype=torch.int32, device=cuda), is_prefill=False)
    cache.prepare_compact_prefill(meta, 12, committed_seq_lens=case["committed"])
    torch.cuda.synchronize()
    state = dict(scores=cache.scores[:12], sel_ids=cache.sel_ids, sel_count=cache.sel_count, plan=cache.plan[:12],
                 work_k=cache.working_key, work_v=cache.working_value)
    check_step(case, state)
    assert cache.working_lens.cpu().tolist() == cache.plan[:12, 1].cpu().tolist()
    if lse_free:
        rows_idx, q_index, _ = O.retrieval_rows(case["counts"], case["ends"], case["tlens"], 12)
        torch.testing.assert_close(cache.scored_lse[rows_idx].cpu(), case["lse"][q_index], rtol=1e-5, atol=1e-4)


def test_runtime_adaptive_cadence_on_device(cuda):
    """adaptive_profile=True on the GPU (diffspec/runtime.py:575-593, fed at :1309-1331): the slot selections
    before and after each retrieval reach pinned host memory on the stream, equal to the device state, and the
    next retrieval call applies the comparison before it reads the interval.  The same snapshot retrieved twice
    keeps every chunk (interval doubled); a different query for the first committed row resets it."""
    from types import SimpleNamespace

    from ds355 import runtime

    g = gen(23)
    rows = 6
    lens = [int(x) for x in torch.randint(6000, 16000, (rows,), generator=g)]
    counts = [3, 1, 4, 2, 5, 1]
    case = build_case(23, real_rows=rows, pad_rows=0, target_lens=lens, query_len=5, counts=counts, hq=32, hkv=4,
                      head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=16000,
                      slots=list(range(rows)), num_slots=rows)

    class Rotary:
        rotary_dim = 128
        is_neox_style = True
        cos_sin_cache = case["cos_sin"].to(cuda)

    settings = runtime.DiffSpecSettings(chunk_size=64, token_budget=2048, retrieval_interval=1, max_tree_nodes=4,
                                        max_tree_depth=4, tree_threshold=0.7, adaptive_profile=True)
    cache = runtime.DiffSpecDraftCache(settings, max_num_reqs=rows, max_model_len=16000, num_kv_heads=4,
                                       head_dim=128, target_num_layers=2, dtype=torch.bfloat16, device=cuda,
                                       rotary_embedding=Rotary())
    ids = [f"request-{i}" for i in range(rows)]
    meta = SimpleNamespace(actual_seq_lengths_q=case["ends"], seq_lens_list=case["tlens"],
                           block_tables=case["table"].to(cuda), num_prefills=0)
    key_cache, lse = case["key_cache"].to(cuda), case["lse"].to(cuda)

    def retrieve(query):
        cache.begin_target_forward(ids)
        cache.capture_target_attention(query, lse, key_cache, meta, case["scale"])
        cache.accept_target_queries(torch.tensor(counts, dtype=torch.int32, device=cuda), is_prefill=False)

    query = case["query"].to(cuda)
    retrieve(query)  # cycle 1: no selection before it
    torch.cuda.synchronize()
    assert torch.equal(cache._adaptive_sel_count[0], torch.full((rows,), -1, dtype=torch.int32))
    assert torch.equal(cache._adaptive_ids[1], cache.sel_ids.cpu())
    assert torch.equal(cache._adaptive_sel_count[1], cache.sel_count.cpu())
    first = cache.sel_ids[0, : int(cache.sel_count[0])].cpu().tolist()
    retrieve(query)  # cycle 2 applies cycle 1 (overlap 0 -> base), then retrieves the same chunks again
    assert cache.retrieval_interval == 1
    cache._observe_previous_retrieval()  # what cycle 3 would apply first: overlap 1, acceptance 2 -> doubled
    assert cache.retrieval_interval == 2
    assert cache.sel_ids[0, : int(cache.sel_count[0])].cpu().tolist() == first
    other = torch.randn(query.shape, generator=torch.Generator().manual_seed(5)).to(query.dtype).to(cuda)
    cache.begin_target_forward(ids)
    cache.capture_target_attention(other, lse, key_cache, meta, case["scale"])
    cache.accept_target_queries(torch.tensor(counts, dtype=torch.int32, device=cuda), is_prefill=False)  # 3 % 2
    assert cache.metrics.retrieval_skipped_interval == 1
    retrieve(other)  # cycle 4: retrieves with the new query
    cache._observe_previous_retrieval()
    changed = cache.sel_ids[0, : int(cache.sel_count[0])].cpu().tolist()
    union, inter = set(first) | set(changed), set(first) & set(changed)
    assert len(inter) / len(union) < 0.9 and cache.retrieval_interval == 1


def test_runtime_populate_prefill_then_compact_prefill(cuda):
    """The proposer's compact-draft-root sequence (proposer.py:256-307) on the GPU:
    accept_target_queries (score + select), begin_cycle, populate_prefill of every
    padded verifier token's projected raw K/V (rejected ones included), then
    prepare_compact_prefill at the committed roots.  Against the oracle's
    write_raw (runtime.py:1602-1618) followed by the per-request CPU rebuild
    (runtime.py:1683-1711) over the same selections: raw caches and working
    caches bit-exact, nothing written past each row's history."""
    from types import SimpleNamespace

    from ds355 import runtime

    g = gen(23)
    rows, qlen, chunk, token_budget, lmax = 6, 5, 32, 1024, 9000
    lens = [int(x) for x in torch.randint(2500, lmax + 1, (rows,), generator=g)]
    counts = [int(x) for x in torch.randint(1, qlen + 1, (rows,), generator=g)]
    case = build_case(23, real_rows=rows, pad_rows=0, target_lens=lens, query_len=qlen, counts=counts, hq=16, hkv=2,
                      head_dim=64, chunk=chunk, token_budget=token_budget, block_size=64, lmax=lmax,
                      slots=list(range(rows)), num_slots=rows)

    class Rotary:
        rotary_dim = 64
        is_neox_style = True
        cos_sin_cache = case["cos_sin"].to(cuda)

    settings = runtime.DiffSpecSettings(chunk_size=chunk, token_budget=token_budget, retrieval_interval=1,
                                        max_tree_nodes=4, max_tree_depth=4, tree_threshold=0.7, adaptive_profile=False)
    cache = runtime.DiffSpecDraftCache(settings, max_num_reqs=rows, max_model_len=lmax, num_kv_heads=2, head_dim=64,
                                       target_num_layers=2, dtype=torch.bfloat16, device=cuda,
                                       rotary_embedding=Rotary())
    cache.raw_key.copy_(case["raw_k"])
    cache.raw_value.copy_(case["raw_v"])
    cache.working_key.fill_(float("nan"))
    cache.working_value.fill_(float("nan"))
    ids = [f"r{i}" for i in range(rows)]
    meta = SimpleNamespace(actual_seq_lengths_q=case["ends"], seq_lens_list=case["tlens"],
                           block_tables=case["table"].to(cuda), num_prefills=0)
    cache.prepare_target_batch(ids, {})
    cache.begin_target_forward(ids)
    cache.capture_target_attention(case["query"].to(cuda), case["lse"].to(cuda), case["key_cache"].to(cuda), meta,
                                   case["scale"])
    cache.accept_target_queries(torch.tensor(counts, dtype=torch.int32, device=cuda), is_prefill=False)
    cache.begin_cycle(ids)
    # The draft's projection of every verifier token: positions target_len - qlen + j.
    positions = [tl - qlen + j for tl in lens for j in range(qlen)]
    key = torch.randn((rows * qlen, 2 * 64), generator=g).to(torch.bfloat16)
    value = torch.randn((rows * qlen, 2, 64), generator=g).to(torch.bfloat16)
    cache.populate_prefill(torch.tensor(positions, dtype=torch.int64, device=cuda), key.to(cuda), value.to(cuda),
                           meta)
    cache.prepare_compact_prefill(meta, rows, committed_seq_lens=case["committed"])
    torch.cuda.synchronize()
    cache.end_cycle()
    assert cache.capture_status() == 0

    raw_k, raw_v = case["raw_k"].clone(), case["raw_v"].clone()
    token_slots = [r for r in range(rows) for _ in range(qlen)]
    O.write_raw(raw_k, raw_v, token_slots, positions, key, value)
    assert torch.equal(cache.raw_key.cpu(), raw_k) and torch.equal(cache.raw_value.cpu(), raw_v)
    # Selections on the GPU's scores (bit-exact selection is checked elsewhere on the same inputs).
    rows_idx, _, lengths = O.retrieval_rows(counts, case["ends"], case["tlens"], rows)
    scores = cache.scores[:rows].cpu()
    budget = O.history_budget(token_budget, 4, chunk)
    selections = {}
    for j, b in enumerate(rows_idx):
        c = (lengths[j] + chunk - 1) // chunk
        sel = O.select_context_chunks(scores[b, :c].contiguous(), lengths[j], chunk, budget)
        selections[b] = sel.token_indices
        assert cache.sel_ids[b, : sel.chunk_indices.numel()].cpu().tolist() == sel.chunk_indices.tolist()
    exp_k = torch.full(tuple(cache.working_key.shape), float("nan"), dtype=torch.bfloat16)
    exp_v = exp_k.clone()
    roots = O.rebuild_working_cache_per_request(raw_k, raw_v, exp_k, exp_v, list(range(rows)), case["committed"],
                                                selections, case["cos_sin"], chunk_size=chunk, budget=budget,
                                                rotary_dim=64, is_neox_style=True)
    assert cache.local_positions.cpu().tolist() == roots
    assert cache.working_lens.cpu().tolist() == roots
    got_k, got_v = cache.working_key.cpu(), cache.working_value.cpu()
    assert torch.equal(got_k.isnan(), exp_k.isnan()) and torch.equal(got_v.isnan(), exp_v.isnan())
    assert torch.equal(torch.nan_to_num(got_k), torch.nan_to_num(exp_k))
    assert torch.equal(torch.nan_to_num(got_v), torch.nan_to_num(exp_v))


def test_runtime_reused_launches_equal_fresh_ones(cuda):
    """The runtime keeps validated launch arguments per layout and refreshes only
    buffer addresses.  Three verify + draft cycles with new activation tensors
    each time (same shapes, new addresses) give bit for bit what a cache that
    validates every call from scratch gives."""
    from types import SimpleNamespace

    from ds355 import runtime

    g = gen(29)
    rows, qlen = 9, 5
    lens = [int(x) for x in torch.randint(3000, 12000, (rows,), generator=g)]
    case = build_case(29, real_rows=rows, pad_rows=0, target_lens=lens, query_len=qlen, counts=[1] * rows, hq=32,
                      hkv=4, head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=12000,
                      slots=list(range(rows)), num_slots=rows)

    class Rotary:
        rotary_dim = 128
        is_neox_style = True
        cos_sin_cache = case["cos_sin"].to(cuda)

    settings = runtime.DiffSpecSettings(chunk_size=64, token_budget=2048, retrieval_interval=1, max_tree_nodes=4,
                                        max_tree_depth=4, tree_threshold=0.7, adaptive_profile=False,
                                        recent_window=256)
    caches = []
    for _ in range(2):
        c = runtime.DiffSpecDraftCache(settings, max_num_reqs=rows, max_model_len=12000, num_kv_heads=4,
                                       head_dim=128, target_num_layers=2, dtype=torch.bfloat16, device=cuda,
                                       rotary_embedding=Rotary())
        c.raw_key.copy_(case["raw_k"])
        c.raw_value.copy_(case["raw_v"])
        c.working_key.zero_()
        c.working_value.zero_()
        caches.append(c)
    fresh = caches[1]

    class NoStore(dict):
        def __setitem__(self, key, value):  # every call validates from scratch
            pass

    fresh._step_descs, fresh._attention_reuse, fresh._capture_reuse = NoStore(), NoStore(), NoStore()
    ids = [f"r{i}" for i in range(rows)]
    meta = SimpleNamespace(actual_seq_lengths_q=case["ends"], seq_lens_list=case["tlens"],
                           block_tables=case["table"].to(cuda), num_prefills=0)
    key_cache = case["key_cache"].to(cuda)
    for cycle in range(3):
        q = torch.randn((case["ends"][-1], 32, 128), generator=g).to(torch.bfloat16)
        lse = case["lse"] + 0.1 * cycle
        counts = torch.randint(1, qlen + 1, (rows,), generator=g).to(torch.int32)
        dq = torch.randn((2, rows, 32, 128), generator=g).to(torch.bfloat16)
        dk = torch.randn((2, rows, 4 * 128), generator=g).to(torch.bfloat16)
        dv = torch.randn((2, rows, 4, 128), generator=g).to(torch.bfloat16)
        pos = [tl - qlen + int(c) for tl, c in zip(lens, counts)]
        outs = []
        for c in caches:
            c.begin_target_forward(ids)
            c.capture_target_attention(q.to(cuda), lse.to(cuda), key_cache, meta, case["scale"])
            c.accept_target_queries(counts.to(cuda), is_prefill=False)
            c.begin_cycle(ids)
            c.prepare_compact_prefill(meta, rows, committed_seq_lens=[p + 1 for p in pos])
            o = []
            for s in range(2):
                if s:
                    c.prepare_draft_step()
                absolute = torch.tensor([p + s for p in pos], dtype=torch.int64, device=cuda)
                rope = c.capture_raw_kv(0, absolute, dk[s].to(cuda), dv[s].to(cuda))
                out = torch.empty((rows, 32 * 128), dtype=torch.bfloat16, device=cuda)
                c.forward_attention(dq[s].to(cuda), dk[s].to(cuda), dv[s].to(cuda), case["scale"], out)
                o.append((rope.clone(), out))
            c.end_cycle()
            outs.append(o)
        torch.cuda.synchronize()
        reused = caches[0]
        for name in ("scores", "sel_ids", "sel_count", "plan", "working_lens", "working_key", "working_value",
                     "raw_key", "raw_value"):
            assert torch.equal(getattr(reused, name), getattr(fresh, name)), (cycle, name)
        for (ra, oa), (rb, ob) in zip(*outs):
            assert torch.equal(ra, rb) and torch.equal(oa, ob), cycle
    assert len(caches[0]._step_descs) == 2 and len(caches[0]._attention_reuse) >= 1
