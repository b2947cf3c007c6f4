"""GPU parity: the compact prefill (the PLAN stage of ds_retrieval_step).

The runtime's prepare_compact_prefill runs plans and gather from the slots'
stored selections (diffspec/runtime.py:1737-1765, compact_kv.py:8-242).  On
the vector path they are one launch (plan_gather_kernel: every workgroup
derives its row's plan from the selection state, workgroup 0 of a row
stores it); other shapes run the plan kernel and the gather.  Every case is
checked against the oracle's plans (runtime.py:1713-1735) and rebuild
(compact_kv.py:8-133), and against ds_build_plan + ds_rebuild_compact_kv on
the same state: plans, working lengths and working caches bit-exact, with
NaN sentinels proving nothing outside [slot, :, 0:history_len] of re-gathered
rows is written.  Selection states mix no selection (-1), empty selections,
short and full selections, with ends before, inside and after the selected
chunks; rows are permuted, padded (slot -1 or out of range) and partly
flagged as reused.
"""

import random

import pytest
import torch

from helpers import O

pytestmark = pytest.mark.gpu


def _state(seed, *, rows, num_slots, chunk, token_budget, hb, heads, head_dim, lmax, dtype):
    rng = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    cap = token_budget // chunk
    sel_ids = torch.zeros((num_slots, cap), dtype=torch.int32)
    sel_count = torch.full((num_slots,), -1, dtype=torch.int32)
    selections = {}
    slots = list(range(num_slots))
    rng.shuffle(slots)
    slots = slots[:rows]
    committed = []
    for i, slot in enumerate(slots):
        end = rng.randint(0, lmax - 1)
        kind = i % 4
        if kind == 0:
            chunks = None
        elif kind == 1:
            chunks = []
        else:
            retrieval_end = max(1, min(lmax, end + rng.randint(-3 * chunk, 3 * chunk)))
            scores = torch.rand((retrieval_end + chunk - 1) // chunk, generator=g)
            chunks = O.select_context_chunks(scores, retrieval_end, chunk, hb).chunk_indices.tolist()
        selections[slot] = chunks
        if chunks is not None:
            sel_count[slot] = len(chunks)
            sel_ids[slot, : len(chunks)] = torch.tensor(chunks, dtype=torch.int32)
        committed.append(end + 1)
    raw_k = torch.randn((num_slots, lmax, heads, head_dim), generator=g).to(dtype)
    raw_v = torch.randn((num_slots, lmax, heads, head_dim), generator=g).to(dtype)
    return dict(sel_ids=sel_ids, sel_count=sel_count, slots=slots, committed=committed, selections=selections,
                raw_k=raw_k, raw_v=raw_v)


def _run(st, device, *, pad, row_active, chunk, token_budget, hb, window, rot, neox, dtype, split):
    """PLAN through ds_retrieval_step (split=False) or ds_build_plan + ds_rebuild_compact_kv (split=True)."""
    from ds355 import plan as plan_mod
    from ds355 import step
    from ds355.compact_kv import rebuild_compact_kv_from_plan

    num_slots, _, heads, head_dim = st["raw_k"].shape
    slots = st["slots"] + pad
    committed = st["committed"] + [5] * len(pad)
    rows = len(slots)
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=device)  # noqa: E731
    work = torch.full((num_slots, heads, token_budget, head_dim), float("nan"), dtype=dtype, device=device)
    out = dict(work_k=work, work_v=work.clone(),
               plan=torch.full((rows, 5 + token_budget // chunk), -3, dtype=torch.int64, device=device),
               working_lens=torch.full((num_slots,), -7, dtype=torch.int32, device=device))
    raw_k, raw_v = st["raw_k"].to(device), st["raw_v"].to(device)
    cos_sin = O.rope_cos_sin_cache(rot, token_budget).to(dtype).to(device) if rot else torch.zeros(
        (token_budget, 2), dtype=dtype, device=device)
    active = None if row_active is None else i32(row_active + [1] * len(pad))
    if split:
        plan = plan_mod.build_history_plans(
            st["sel_ids"].to(device), st["sel_count"].to(device), i32(slots), i32(committed), chunk_size=chunk,
            history_budget=hb, token_budget=token_budget, recent_window=window, working_lens=out["working_lens"])
        out["plan"].copy_(plan)
        rebuild_compact_kv_from_plan(raw_k, raw_v, out["work_k"], out["work_v"], out["plan"], cos_sin,
                                     chunk_size=chunk, max_width=hb, rotary_dim=rot, is_neox_style=neox,
                                     row_active=active)
    else:
        step.retrieval_step(
            stages=step.PLAN, snapshot=None, rows=None, scores=None, sel_ids=st["sel_ids"].to(device),
            sel_count=st["sel_count"].to(device), slots=i32(slots), committed_lens=i32(committed), plan=out["plan"],
            working_lens=out["working_lens"], raw_key=raw_k, raw_value=raw_v, working_key=out["work_k"],
            working_value=out["work_v"], cos_sin_cache=cos_sin, rotary_dim=rot, is_neox_style=neox,
            chunk_size=chunk, history_budget=hb, recent_window=window, row_active=active)
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in out.items()}


def _check(st, got, *, pad, row_active, chunk, token_budget, hb, window, rot, neox, dtype):
    num_slots, _, heads, head_dim = st["raw_k"].shape
    plans = [O.history_plan(s, st["selections"][s], c - 1, chunk, hb, window)
             for s, c in zip(st["slots"], st["committed"])] + [[0, 0, 0, 0, 0]] * len(pad)
    expected_plan = O.pad_plan(plans, token_budget, chunk)
    assert torch.equal(got["plan"], expected_plan)
    lens = got["working_lens"].tolist()
    for s in range(num_slots):
        expect = next((p[1] for p in plans if p[0] == s and s in st["slots"]), -7)
        assert lens[s] == expect, s
    exp_k = torch.full((num_slots, heads, token_budget, head_dim), float("nan"), dtype=dtype)
    exp_v = exp_k.clone()
    cos_sin = O.rope_cos_sin_cache(rot, token_budget).to(dtype) if rot else torch.zeros((token_budget, 2), dtype=dtype)
    O.rebuild_compact_kv_from_plan(st["raw_k"], st["raw_v"], exp_k, exp_v, expected_plan[: len(st["slots"])],
                                   cos_sin, chunk_size=chunk, max_width=hb, rotary_dim=rot, is_neox_style=neox,
                                   row_active=row_active)
    for key, exp in (("work_k", exp_k), ("work_v", exp_v)):
        assert torch.equal(got[key].isnan(), exp.isnan()), key
        assert torch.equal(torch.nan_to_num(got[key]), torch.nan_to_num(exp)), key


CASES = [
    # chunk, token_budget, window, heads, head_dim, rot, neox, dtype
    (64, 2048, 256, 4, 128, 128, True, torch.bfloat16),
    (32, 2048, 64, 4, 128, 128, True, torch.bfloat16),
    (128, 4096, 512, 8, 128, 128, True, torch.bfloat16),
    (16, 2048, 48, 2, 64, 64, False, torch.float16),
    (64, 1024, 64, 2, 256, 128, True, torch.bfloat16),
    (32, 1024, 96, 1, 128, 64, False, torch.float32),
    (64, 1024, 128, 2, 96, 96, True, torch.bfloat16),  # 6 lanes per position: lanes 60..63 idle
    (8, 2048, 8, 2, 64, 64, True, torch.bfloat16),     # 256 chunk ids per row: plan kernel + gather
    (64, 1024, 128, 2, 72, 72, True, torch.bfloat16),  # head_dim 72: plan kernel + scalar gather
    (64, 1024, 128, 3, 128, 128, False, torch.float16),  # heads in pairs, then one alone
    (32, 2048, 64, 7, 64, 64, True, torch.bfloat16),     # heads in fours, then three
]


@pytest.mark.parametrize("chunk,token_budget,window,heads,head_dim,rot,neox,dtype", CASES)
def test_compact_prefill_matches_oracle_and_split_path(cuda, chunk, token_budget, window, heads, head_dim, rot, neox,
                                                       dtype):
    hb = O.history_budget(token_budget, 4, chunk)
    lmax = 6000
    print(f"compact prefill: chunk {chunk}, budget {token_budget} (history {hb}), window {window}, "
          f"{heads} x {head_dim}, rot {rot}, {'neox' if neox else 'gptj'}, {dtype}", flush=True)
    st = _state(chunk + head_dim, rows=11, num_slots=13, chunk=chunk, token_budget=token_budget, hb=hb, heads=heads,
                head_dim=head_dim, lmax=lmax, dtype=dtype)
    pad = [-1, 13]
    row_active = [1, 1, 0, 1, 1, 1, 0, 1, 1, 1, 1]
    kw = dict(pad=pad, row_active=row_active, chunk=chunk, token_budget=token_budget, hb=hb, window=window, rot=rot,
              neox=neox, dtype=dtype)
    one = _run(st, cuda, split=False, **kw)
    _check(st, one, **kw)
    two = _run(st, cuda, split=True, **kw)
    for key in one:
        a, b = one[key], two[key]
        if a.dtype.is_floating_point:
            assert torch.equal(a.isnan(), b.isnan()) and torch.equal(torch.nan_to_num(a), torch.nan_to_num(b)), key
        else:
            assert torch.equal(a, b), key


def test_compact_prefill_all_rows_without_reuse_flags(cuda):
    """No row_active: every real row re-gathered; long histories reach the budget."""
    chunk, token_budget, window = 64, 2048, 256
    hb = O.history_budget(token_budget, 4, chunk)
    st = _state(3, rows=16, num_slots=16, chunk=chunk, token_budget=token_budget, hb=hb, heads=4, head_dim=128,
                lmax=40000, dtype=torch.bfloat16)
    kw = dict(pad=[], row_active=None, chunk=chunk, token_budget=token_budget, hb=hb, window=window, rot=128,
              neox=True, dtype=torch.bfloat16)
    _check(st, _run(st, cuda, split=False, **kw), **kw)
