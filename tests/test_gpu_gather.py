"""GPU parity: gather + local RoPE + working-cache write (ds_rebuild_compact_kv).

Mirrors the reference's batched-rebuild device test
(tests/test_linear_attention_batch_npu.py:20-71): the batched rebuild must be
bit-equal to the per-request path, unused slots stay NaN and the raw caches
are unchanged.  The expected values come from the CPU oracle.
"""

import pytest
import torch

from helpers import O, gen, max_ulp_bf16, randn, rope_table_recipe

pytestmark = pytest.mark.gpu


def _run_batched(cache_k, cache_v, work_k, work_v, plan, cos_sin, chunk, width, rot, neox, device, row_active=None):
    from ds355.compact_kv import rebuild_compact_kv_from_plan

    rebuild_compact_kv_from_plan(
        cache_k, cache_v, work_k, work_v, plan.to(device), cos_sin.to(device),
        chunk_size=chunk, max_width=width, rotary_dim=rot, is_neox_style=neox,
        row_active=None if row_active is None else row_active.to(device),
    )


@pytest.mark.parametrize("heads,dim,rotary_dim,neox", [
    (2, 128, 128, True),
    (4, 256, 256, True),
    (4, 256, 128, True),
    (2, 128, 64, False),
    (3, 128, 128, True),   # heads in pairs, then one alone
    (5, 64, 64, False),    # heads in fours, then one alone
])
@pytest.mark.parametrize("slots", [[0, 1], [2, 0]])
def test_batched_rebuild_matches_per_request_path(cuda, heads, dim, rotary_dim, neox, slots):
    chunk, token_budget, depth = 8, 64, 4
    budget = O.history_budget(token_budget, depth, chunk)
    g = gen(17)
    raw_k = randn((3, 128, heads, dim), torch.bfloat16, g)
    raw_v = randn((3, 128, heads, dim), torch.bfloat16, g)
    cos_sin = rope_table_recipe(rotary_dim)
    dev_raw_k, dev_raw_v = raw_k.to(cuda), raw_v.to(cuda)
    work_k = torch.full((3, heads, token_budget, dim), float("nan"), dtype=torch.bfloat16, device=cuda)
    work_v = torch.full_like(work_k, float("nan"))
    for end in [0, 1, 7, 62, 66, 73]:
        selections = {}
        for slot in slots:
            sel = O.select_context_chunks(torch.arange((end + 7) // 8, dtype=torch.float32), end, chunk, budget)
            selections[slot] = sel.token_indices
        lengths = [end + 1, end + 6]
        exp_k = torch.full((3, heads, token_budget, dim), float("nan"), dtype=torch.bfloat16)
        exp_v = exp_k.clone()
        expected_lens = O.rebuild_working_cache_per_request(
            raw_k, raw_v, exp_k, exp_v, slots, lengths, selections, cos_sin,
            chunk_size=chunk, budget=budget, rotary_dim=rotary_dim, is_neox_style=neox,
        )
        plans = []
        for slot, n in zip(slots, lengths):
            tokens = selections[slot]
            chunks = sorted({int(t) // chunk for t in tokens[::chunk]}) if tokens.numel() else []
            plans.append(O.history_plan(slot, chunks if tokens is not None else None, max(0, n - 1), chunk, budget))
        plan = O.pad_plan(plans, token_budget, chunk)
        width = max(p[1] for p in plans)
        assert [p[1] for p in plans] == expected_lens
        if width:
            _run_batched(dev_raw_k, dev_raw_v, work_k, work_v, plan, cos_sin, chunk, width, rotary_dim, neox, cuda)
        got_k, got_v = work_k.cpu(), work_v.cpu()
        for slot, n in zip(slots, expected_lens):
            # The per-request path is the batched path's specification: bit-equal.
            assert torch.equal(got_k[slot, :, :n], exp_k[slot, :, :n]), (end, slot)
            assert torch.equal(got_v[slot, :, :n], exp_v[slot, :, :n]), (end, slot)
        for unused in set(range(3)) - set(slots):
            assert torch.isnan(got_k[unused]).all()
            assert torch.isnan(got_v[unused]).all()
    assert torch.equal(dev_raw_k.cpu(), raw_k)
    assert torch.equal(dev_raw_v.cpu(), raw_v)


def _random_plans(g, rows, slots, chunk, budget, token_budget, max_len):
    plans = []
    for r in range(rows):
        end = int(torch.randint(1, max_len, (1,), generator=g))
        c = (end + 1 + chunk - 1) // chunk
        scores = torch.rand(c, generator=g)
        sel = O.select_context_chunks(scores, end + 1, chunk, budget)
        plans.append(O.history_plan(slots[r], sel.chunk_indices.tolist(), end, chunk, budget))
    return plans


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("neox,rotary_dim", [(True, 128), (True, 64), (False, 128), (True, 0)])
def test_gather_dtypes_and_layouts(cuda, dtype, neox, rotary_dim):
    chunk, token_budget, depth, heads, dim, lmax = 64, 2048, 4, 4, 128, 6000
    budget = O.history_budget(token_budget, depth, chunk)
    g = gen(5)
    slots = [3, 0, 5, 1]
    raw_k = randn((6, lmax, heads, dim), dtype, g)
    raw_v = randn((6, lmax, heads, dim), dtype, g)
    cos_sin = O.rope_cos_sin_cache(max(rotary_dim, 2), token_budget, dtype=dtype)[:, : max(rotary_dim, 2)]
    plans = _random_plans(g, 4, slots, chunk, budget, token_budget, lmax - 1)
    plan = O.pad_plan(plans, token_budget, chunk)
    width = max(p[1] for p in plans)
    exp_k = torch.full((6, heads, token_budget, dim), float("nan"), dtype=dtype)
    exp_v = exp_k.clone()
    O.rebuild_compact_kv_from_plan(raw_k, raw_v, exp_k, exp_v, plan, cos_sin, chunk_size=chunk,
                                   max_width=width, rotary_dim=rotary_dim, is_neox_style=neox)
    work_k = torch.full_like(exp_k, float("nan")).to(cuda)
    work_v = torch.full_like(exp_v, float("nan")).to(cuda)
    _run_batched(raw_k.to(cuda), raw_v.to(cuda), work_k, work_v, plan, cos_sin, chunk, width, rotary_dim, neox, cuda)
    got_k, got_v = work_k.cpu(), work_v.cpu()
    assert torch.equal(got_v.isnan(), exp_v.isnan())
    assert torch.equal(torch.nan_to_num(got_v), torch.nan_to_num(exp_v))
    # Rotated K: fp32 maths rounded once, bit-exact with the oracle (<= 1 bf16 ulp is the contract).
    assert torch.equal(got_k.isnan(), exp_k.isnan())
    assert torch.equal(torch.nan_to_num(got_k), torch.nan_to_num(exp_k))


def test_gather_scalar_fallback_matches_oracle(cuda):
    """Shapes the 16-byte path does not cover (head_dim 6, rotary 2..6) take the element path."""
    g = gen(9)
    chunk, token_budget = 2, 8
    budget = O.history_budget(token_budget, 2, chunk)
    for dim, rot, neox in [(6, 6, True), (6, 4, False), (6, 2, True), (2, 2, True)]:
        raw_k = randn((2, 16, 1, dim), torch.float32, g)
        raw_v = randn((2, 16, 1, dim), torch.float32, g)
        cos_sin = rope_table_recipe(rot, rows=16, dtype=torch.float32)
        plans = [O.history_plan(1, [0, 2, 4], 9, chunk, budget), O.history_plan(0, None, 5, chunk, budget)]
        plan = O.pad_plan(plans, token_budget, chunk)
        width = max(p[1] for p in plans)
        exp_k = torch.full((2, 1, token_budget, dim), float("nan"))
        exp_v = exp_k.clone()
        O.rebuild_compact_kv_from_plan(raw_k, raw_v, exp_k, exp_v, plan, cos_sin, chunk_size=chunk,
                                       max_width=width, rotary_dim=rot, is_neox_style=neox)
        work_k = torch.full_like(exp_k, float("nan")).to(cuda)
        work_v = torch.full_like(exp_v, float("nan")).to(cuda)
        _run_batched(raw_k.to(cuda), raw_v.to(cuda), work_k, work_v, plan, cos_sin, chunk, width, rot, neox, cuda)
        assert torch.equal(torch.nan_to_num(work_k.cpu(), 7.0), torch.nan_to_num(exp_k, 7.0)), (dim, rot, neox)
        assert torch.equal(torch.nan_to_num(work_v.cpu(), 7.0), torch.nan_to_num(exp_v, 7.0)), (dim, rot, neox)


def test_reference_value_kat(cuda):
    """tests/test_runtime.py:781-803: values carry their absolute position."""
    cases = [
        (list(range(65)), 64, list(range(64))),
        (list(range(70)), 64, list(range(64))),
        (list(range(32)) + list(range(96, 128)), 127, list(range(32)) + list(range(95, 127))),
        (list(range(12)), 11, list(range(11))),
    ]
    chunk, token_budget = 32, 128
    budget = O.history_budget(token_budget, 3, chunk)
    raw_k = torch.zeros((1, 256, 1, 32), dtype=torch.float32)
    raw_v = torch.zeros_like(raw_k)
    raw_k[0, :, 0, 0] = torch.arange(256)
    raw_v[0, :, 0, 0] = torch.arange(256) + 1000
    for selected, end, expected in cases:
        tokens = torch.tensor(selected)
        assert O.history_indices(tokens, end, chunk, budget).tolist() == expected
        chunks = sorted({t // chunk for t in selected[::chunk]})
        plan = O.pad_plan([O.history_plan(0, chunks, end, chunk, budget)], token_budget, chunk)
        work_k = torch.full((1, 1, token_budget, 32), float("nan"), device=cuda)
        work_v = torch.full_like(work_k, float("nan"))
        cos_sin = torch.zeros((token_budget, 2))
        _run_batched(raw_k.to(cuda), raw_v.to(cuda), work_k, work_v, plan, cos_sin, chunk, len(expected), 0, True, cuda)
        assert work_k[0, 0, : len(expected), 0].cpu().tolist() == expected
        assert work_v[0, 0, : len(expected), 0].cpu().tolist() == [p + 1000 for p in expected]


def test_row_active_and_width_limit(cuda):
    chunk, token_budget, heads, dim = 64, 2048, 4, 128
    budget = O.history_budget(token_budget, 4, chunk)
    g = gen(11)
    raw_k = randn((4, 8192, heads, dim), torch.bfloat16, g)
    raw_v = randn((4, 8192, heads, dim), torch.bfloat16, g)
    cos_sin = O.rope_cos_sin_cache(dim, token_budget)
    plans = _random_plans(g, 4, [0, 1, 2, 3], chunk, budget, token_budget, 8000)
    plan = O.pad_plan(plans, token_budget, chunk)
    width = max(p[1] for p in plans)
    active = torch.tensor([1, 0, 1, 0], dtype=torch.int32)
    exp_k = torch.full((4, heads, token_budget, dim), float("nan"), dtype=torch.bfloat16)
    exp_v = exp_k.clone()
    O.rebuild_compact_kv_from_plan(raw_k, raw_v, exp_k, exp_v, plan, cos_sin, chunk_size=chunk, max_width=width,
                                   rotary_dim=dim, is_neox_style=True, row_active=[bool(x) for x in active])
    work_k = torch.full_like(exp_k, float("nan")).to(cuda)
    work_v = torch.full_like(exp_v, float("nan")).to(cuda)
    _run_batched(raw_k.to(cuda), raw_v.to(cuda), work_k, work_v, plan, cos_sin, chunk, width, dim, True, cuda,
                 row_active=active)
    assert torch.equal(torch.nan_to_num(work_k.cpu()), torch.nan_to_num(exp_k))
    assert torch.equal(torch.nan_to_num(work_v.cpu()), torch.nan_to_num(exp_v))
    assert torch.isnan(work_k[1]).all() and torch.isnan(work_k[3]).all()


def test_headline_shape_gather_bit_exact(cuda):
    """16 rows of a 40k-token raw cache, 4 KV heads x 128, chunk 64, budget 2048."""
    chunk, token_budget, heads, dim, lmax = 64, 2048, 4, 128, 40960
    budget = O.history_budget(token_budget, 4, chunk)
    g = gen(2)
    raw_k = randn((16, lmax, heads, dim), torch.bfloat16, g)
    raw_v = randn((16, lmax, heads, dim), torch.bfloat16, g)
    cos_sin = O.rope_cos_sin_cache(dim, token_budget)
    plans = _random_plans(g, 16, list(range(16)), chunk, budget, token_budget, lmax - 1)
    plan = O.pad_plan(plans, token_budget, chunk)
    width = max(p[1] for p in plans)
    exp_k = torch.zeros((16, heads, token_budget, dim), dtype=torch.bfloat16)
    exp_v = exp_k.clone()
    O.rebuild_compact_kv_from_plan(raw_k, raw_v, exp_k, exp_v, plan, cos_sin, chunk_size=chunk, max_width=width,
                                   rotary_dim=dim, is_neox_style=True)
    work_k = torch.zeros_like(exp_k).to(cuda)
    work_v = torch.zeros_like(exp_v).to(cuda)
    _run_batched(raw_k.to(cuda), raw_v.to(cuda), work_k, work_v, plan, cos_sin, chunk, width, dim, True, cuda)
    got_k = work_k.cpu()
    assert torch.equal(work_v.cpu(), exp_v)
    assert max_ulp_bf16(got_k, exp_k) <= 1
    assert torch.equal(got_k, exp_k)


def test_validation_messages_match_reference(cuda):
    from ds355.compact_kv import rebuild_compact_kv_from_plan

    k = torch.zeros((2, 8, 1, 16), dtype=torch.bfloat16, device=cuda)
    w = torch.zeros((2, 1, 8, 16), dtype=torch.bfloat16, device=cuda)
    plan = torch.zeros((1, 5 + 8 // 2), dtype=torch.int64, device=cuda)
    cs = torch.zeros((8, 16), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="rotary_dim must be even"):
        rebuild_compact_kv_from_plan(k, k, w, w, plan, cs, chunk_size=2, max_width=4, rotary_dim=3, is_neox_style=True)
    with pytest.raises(ValueError, match="plan width must be 5"):
        rebuild_compact_kv_from_plan(k, k, w, w, plan, cs, chunk_size=4, max_width=4, rotary_dim=16, is_neox_style=True)
    with pytest.raises(ValueError, match="KV plan must be a contiguous 2-D int64"):
        rebuild_compact_kv_from_plan(k, k, w, w, plan.int(), cs, chunk_size=2, max_width=4, rotary_dim=16,
                                     is_neox_style=True)


def _special_keys(g, n, heads, dim, cos_sin, rot):
    """bf16 keys that probe the rotation's rounding: ordinary values, signed
    zeros, NaN and infinities, values near the top of the range, tiny normal
    values, near-cancelling pairs (x1*c ~ x2*s) and a wide exponent spread."""
    x = torch.randn((n, heads, dim), generator=g)
    kind = torch.arange(n) % 8
    half = rot // 2
    sign = torch.where(torch.rand((n, heads, dim), generator=g) < 0.5, -1.0, 1.0)
    for p in range(n):
        k = int(kind[p])
        if k == 1:
            x[p][torch.rand((heads, dim), generator=g) < 0.5] = 0.0
            x[p] *= sign[p]
        elif k == 2:
            pick = torch.randint(0, 4, (heads, dim), generator=g)
            x[p][pick == 1] = float("nan")
            x[p][pick == 2] = float("inf")
            x[p][pick == 3] = float("-inf")
        elif k == 3:
            x[p] = sign[p] * torch.empty((heads, dim)).uniform_(1e37, 3.3e38, generator=g)
        elif k == 4:
            x[p] = sign[p] * torch.empty((heads, dim)).uniform_(1e-30, 1e-28, generator=g)
        elif k == 5:
            c = cos_sin[p, :half].float()
            s = cos_sin[p, half:rot].float()
            first = x[p, :, :half].to(torch.bfloat16).float()
            ok = s.abs() > 1e-3
            second = torch.where(ok, first * c / torch.where(ok, s, torch.ones_like(s)), x[p, :, half:rot])
            x[p, :, half:rot] = second
        elif k == 7:
            x[p] = sign[p] * torch.exp2(torch.empty((heads, dim)).uniform_(-60, 60, generator=g))
    return x.to(torch.bfloat16)


def test_rotation_special_values_bit_exact(cuda):
    """Every rotated word that is not a NaN equals the oracle's bit for bit
    (signed zeros included), and NaNs sit in the same places, for neox and
    GPT-J pairs, on keys built to probe the fp32 rotation's rounding
    (_special_keys).  NaN payloads are not compared: the oracle's conversion
    keeps whatever NaN bits the host CPU produced, the kernel writes 0x7fc0."""
    from ds355.compact_kv import rebuild_compact_kv_from_plan

    chunk, token_budget, heads, dim, n = 64, 2048, 4, 128, 512
    budget = O.history_budget(token_budget, 4, chunk)
    g = gen(29)
    cos_sin = O.rope_cos_sin_cache(dim, token_budget)
    for neox in (True, False):
        raw_k = _special_keys(g, n + 1, heads, dim, cos_sin, dim).unsqueeze(0)
        raw_v = randn((1, n + 1, heads, dim), torch.bfloat16, g)
        plan = O.pad_plan([O.history_plan(0, None, n, chunk, budget)], token_budget, chunk)
        width = int(plan[0, 1])
        exp_k = torch.zeros((1, heads, token_budget, dim), dtype=torch.bfloat16)
        exp_v = exp_k.clone()
        O.rebuild_compact_kv_from_plan(raw_k, raw_v, exp_k, exp_v, plan, cos_sin, chunk_size=chunk,
                                       max_width=width, rotary_dim=dim, is_neox_style=neox)
        work_k = torch.zeros_like(exp_k).to(cuda)
        work_v = torch.zeros_like(exp_v).to(cuda)
        rebuild_compact_kv_from_plan(raw_k.to(cuda), raw_v.to(cuda), work_k, work_v, plan.to(cuda),
                                     cos_sin.to(cuda), chunk_size=chunk, max_width=width, rotary_dim=dim,
                                     is_neox_style=neox)
        got_nan, want_nan = work_k.cpu().isnan(), exp_k.isnan()
        assert torch.equal(got_nan, want_nan), neox
        got = work_k.cpu().view(torch.int16).masked_fill(got_nan, 0)
        want = exp_k.view(torch.int16).masked_fill(want_nan, 0)
        bad = (got != want).nonzero()
        assert bad.numel() == 0, (neox, bad[:8].tolist(), got[tuple(bad[0])].item(), want[tuple(bad[0])].item())
        assert torch.equal(work_v.cpu().view(torch.int16), exp_v.view(torch.int16))
