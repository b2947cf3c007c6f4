"""GPU: linear draft attention over the working cache against the oracle.

Mirrors the reference's device test of batched draft attention
(tests/test_linear_attention_batch_npu.py:74-144): canonical slots in order
and permuted, NaN beyond every row's position, two consecutive draft steps,
output rows past the batch zero, working lengths advanced.  Every launch is
also checked against the oracle (diffspec/runtime.py:2024-2077): the working
caches bit for bit (the new key/value rows are copies), the output within
one bf16/fp16 rounding of the oracle's fp32 result, and within the
reference's own tolerance (rtol 0.03, atol 0.02) of its expectation.
"""

import pytest
import torch

from helpers import assert_attention_close, attention_terms, gen, randn
from oracle import diffspec_oracle as O

pytestmark = pytest.mark.gpu

REF_RTOL, REF_ATOL = 0.03, 0.02


def _same_bits(a, b):
    assert torch.equal(a.isnan(), b.isnan())
    assert torch.equal(torch.nan_to_num(a), torch.nan_to_num(b))


class Case:
    """Working caches with NaN past every slot's valid prefix, plus per-step inputs."""

    def __init__(self, seed, num_slots, hkv, hq, head_dim, budget, dtype=torch.bfloat16):
        self.g = gen(seed)
        self.shape = (num_slots, hkv, budget, head_dim)
        self.work_k = torch.full(self.shape, float("nan"), dtype=dtype)
        self.work_v = self.work_k.clone()
        self.lens = torch.zeros(num_slots, dtype=torch.int32)
        self.hkv, self.hq, self.head_dim, self.budget, self.dtype = hkv, hq, head_dim, budget, dtype

    def fill(self, slot, length):
        self.work_k[slot, :, :length] = randn((self.hkv, length, self.head_dim), self.dtype, self.g)
        self.work_v[slot, :, :length] = randn((self.hkv, length, self.head_dim), self.dtype, self.g)
        self.lens[slot] = length

    def inputs(self, tokens):
        q = randn((tokens, self.hq, self.head_dim), self.dtype, self.g)
        k = randn((tokens, self.hkv, self.head_dim), self.dtype, self.g)
        v = randn((tokens, self.hkv, self.head_dim), self.dtype, self.g)
        return q, k, v


class Device:
    def __init__(self, case, cuda, rows):
        from ds355 import attention

        self.k = case.work_k.to(cuda)
        self.v = case.work_v.to(cuda)
        self.lens = case.lens.to(cuda)
        self.ws = attention.new_attention_workspace(rows, case.hq, case.hkv, case.head_dim, case.budget, cuda)


def _step(case, dev, cuda, slots, positions, tokens, scale, device_positions=False):
    """One launch and the oracle on the same inputs; returns the GPU output."""
    from ds355 import attention

    q, k, v = case.inputs(tokens)
    if positions is None:
        host_pos = [int(case.lens[s]) for s in slots]
        pos_arg = None
    else:
        host_pos = list(positions)
        pos_arg = torch.tensor(host_pos, dtype=torch.int32, device=cuda) if device_positions else host_pos
    expected = torch.full_like(q, float("nan"))
    lens = case.lens.tolist()
    O.draft_linear_attention(q, k, v, scale, expected, case.work_k, case.work_v, lens, slots, host_pos)
    case.lens = torch.tensor(lens, dtype=torch.int32)
    out = torch.full_like(q, float("nan")).to(cuda)
    attention.draft_linear_attention(q.to(cuda), k.to(cuda), v.to(cuda), out, dev.k, dev.v, dev.lens, slots, pos_arg,
                                     scale=scale, workspace=dev.ws)
    torch.cuda.synchronize()
    actual = out.cpu()
    rows = len(slots)
    terms = attention_terms(q[:rows], case.work_k, case.work_v, slots, host_pos, scale)
    assert_attention_close(actual[:rows], expected[:rows], terms)
    assert actual[rows:].count_nonzero() == 0
    _same_bits(dev.k.cpu(), case.work_k)
    _same_bits(dev.v.cpu(), case.work_v)
    assert torch.equal(dev.lens.cpu(), case.lens)
    assert attention.attention_status(dev.ws) == 0
    return actual, q, k, v, host_pos


@pytest.mark.parametrize("slots", [[0], [0, 1, 2], [3, 0, 2]])
@pytest.mark.parametrize("heads,dim,query_heads", [(2, 128, 8), (4, 256, 4)])
def test_batched_linear_attention_matches_ragged_reference(cuda, slots, heads, dim, query_heads):
    """The reference's device test: budget 64, positions [3, 11, 6], two steps, 5 query rows."""
    case = Case(31, 4, heads, query_heads, dim, 64)
    positions = [3, 11, 6][: len(slots)]
    for s, p in zip(slots, positions):
        case.fill(s, p)
    keys_before = case.work_k.clone()
    values_before = case.work_v.clone()
    dev = Device(case, cuda, 5)
    for step in range(2):
        actual, q, new_k, new_v, _ = _step(case, dev, cuda, slots, [p + step for p in positions], 5, dim ** -0.5)
        for row, (slot, position) in enumerate(zip(slots, positions)):
            end = position + step + 1
            keys_before[slot, :, end - 1] = new_k[row]
            values_before[slot, :, end - 1] = new_v[row]
            k = keys_before[slot, :, :end].repeat_interleave(query_heads // heads, dim=0).float()
            v = values_before[slot, :, :end].repeat_interleave(query_heads // heads, dim=0).float()
            weights = torch.einsum("hd,hsd->hs", q[row].float(), k)
            expected = torch.einsum("hs,hsd->hd", (weights * dim ** -0.5).softmax(-1), v)
            torch.testing.assert_close(actual[row].float(), expected, rtol=REF_RTOL, atol=REF_ATOL)
            assert int(dev.lens[slot]) == end


def test_long_rows_span_merge_and_device_positions(cuda):
    """Budget 2048 with rows ending at span boundaries, permuted slots, then
    two steps that read positions from the slots' working lengths on the device."""
    from ds355 import attention

    case = Case(7, 12, 4, 32, 128, 2048)
    slots = [5, 0, 11, 3, 7, 1, 9, 2]
    lengths = [0, 1, 255, 256, 257, 1000, 1791, 2045]
    for s, n in zip(slots, lengths):
        case.fill(s, n)
    dev = Device(case, cuda, 10)
    _step(case, dev, cuda, slots, lengths, 10, 128 ** -0.5)
    for _ in range(2):
        _step(case, dev, cuda, slots, None, 10, 128 ** -0.5)
    assert attention.attention_epoch(dev.ws) == 3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv,dim", [(8, 8, 64), (16, 2, 128), (64, 2, 128), (24, 2, 64), (8, 1, 256)])
def test_group_sizes_dtypes_and_head_dims(cuda, dtype, hq, hkv, dim):
    """G = 1, 8, 32 (two query blocks) and 12 (a partial block); head_dim 64/128/256; bf16 and fp16."""
    case = Case(hq * 100 + dim, 6, hkv, hq, dim, 1024, dtype)
    slots = [4, 1, 0]
    lengths = [700, 5, 1023 - 1]
    for s, n in zip(slots, lengths):
        case.fill(s, n)
    dev = Device(case, cuda, 3)
    _step(case, dev, cuda, slots, lengths, 3, dim ** -0.5, device_positions=True)
    _step(case, dev, cuda, slots, None, 3, dim ** -0.5)


def test_reused_workspace_across_shapes(cuda):
    """One workspace serves batches of different sizes and layouts one after another."""
    from ds355 import attention

    big = Case(3, 8, 4, 32, 128, 2048)
    for s in range(8):
        big.fill(s, 250 * s + 17)
    dev = Device(big, cuda, 8)
    _step(big, dev, cuda, list(range(8)), None, 8, 0.09)
    small = Case(4, 3, 2, 4, 64, 512)
    for s in range(3):
        small.fill(s, 100 * s + 300)
    dev_small = Device(small, cuda, 3)
    dev_small.ws = dev.ws  # larger than needed: counters and tags carry over
    _step(small, dev_small, cuda, [2, 0], None, 2, 0.2)
    _step(big, dev, cuda, [7, 3, 1], None, 4, 0.09)
    assert attention.attention_epoch(dev.ws) == 3


def test_out_of_range_position_zeroes_the_row_and_sets_status(cuda):
    """A device position past the budget cannot raise on the host: its row is
    zero, nothing else changes for it, the other rows are unaffected, and
    bit 0 of the status word is set."""
    from ds355 import attention

    case = Case(5, 3, 2, 8, 128, 256)
    for s in range(3):
        case.fill(s, 40 + s)
    dev = Device(case, cuda, 3)
    q, k, v = case.inputs(3)
    out = torch.full_like(q, float("nan")).to(cuda)
    pos = torch.tensor([40, 256, 42], dtype=torch.int32, device=cuda)
    attention.draft_linear_attention(q.to(cuda), k.to(cuda), v.to(cuda), out, dev.k, dev.v, dev.lens, [0, 1, 2], pos,
                                     scale=0.1, workspace=dev.ws)
    torch.cuda.synchronize()
    expected = torch.zeros_like(q)
    lens = case.lens.tolist()
    O.draft_linear_attention(q[[0, 2]], k[[0, 2]], v[[0, 2]], 0.1, expected[:2], case.work_k, case.work_v, lens,
                             [0, 2], [40, 42])
    actual = out.cpu()
    terms = attention_terms(q[[0, 2]], case.work_k, case.work_v, [0, 2], [40, 42], 0.1)
    assert_attention_close(actual[[0, 2]], expected[:2], terms)
    assert actual[1].count_nonzero() == 0
    assert dev.lens.cpu().tolist() == [41, 41, 43]
    _same_bits(dev.k.cpu(), case.work_k)
    assert attention.attention_status(dev.ws) & attention.STATUS_BAD_POSITION


def test_runtime_forward_attention_after_compact_prefill(cuda):
    """DiffSpecDraftCache: the rebuild arms the root step at each slot's history
    length; forward_attention then runs on the device state with no host reads."""
    from ds355 import runtime

    class Rotary:
        rotary_dim = 128
        is_neox_style = True

        def __init__(self):
            self.cos_sin_cache = O.rope_cos_sin_cache(128, 512, 1.0e6).to(torch.bfloat16)

    settings = runtime.DiffSpecSettings(chunk_size=16, token_budget=256, retrieval_interval=1, max_tree_nodes=4,
                                        max_tree_depth=4, tree_threshold=0.7, adaptive_profile=False)
    cache = runtime.DiffSpecDraftCache(settings, max_num_reqs=4, max_model_len=512, num_kv_heads=2, head_dim=128,
                                       target_num_layers=2, dtype=torch.bfloat16, device=cuda,
                                       rotary_embedding=Rotary())
    g = gen(21)
    cache.raw_key.copy_(randn(cache.raw_key.shape, torch.bfloat16, g))
    cache.raw_value.copy_(randn(cache.raw_value.shape, torch.bfloat16, g))
    cache.working_key.fill_(float("nan"))
    cache.working_value.fill_(float("nan"))
    cache.set_active_requests(["a", "b", "c"])
    cache.prepare_compact_prefill(None, 3, committed_seq_lens=[300, 40, 7])
    torch.cuda.synchronize()
    work_k, work_v = cache.working_key.cpu(), cache.working_value.cpu()
    lens = cache.working_lens.cpu().tolist()
    for step in range(3):
        if step:
            cache.prepare_draft_step()
        slots = list(cache._pending_request_indices)
        positions = [lens[s] for s in slots]
        q = randn((4, 8, 128), torch.bfloat16, g)
        k = randn((4, 2, 128), torch.bfloat16, g)
        v = randn((4, 2, 128), torch.bfloat16, g)
        expected = torch.empty_like(q)
        O.draft_linear_attention(q, k, v, 0.088, expected, work_k, work_v, lens, slots, positions)
        out = torch.full((4, 8 * 128), float("nan"), dtype=torch.bfloat16, device=cuda)
        cache.forward_attention(q.to(cuda), k.view(4, 256).to(cuda), v.to(cuda), 0.088, out)
        assert not cache.has_pending_attention()
        torch.cuda.synchronize()
        terms = torch.zeros((4, 8, 128))
        terms[: len(slots)] = attention_terms(q[: len(slots)], work_k, work_v, slots, positions, 0.088)
        assert_attention_close(out.view(4, 8, 128).cpu(), expected, terms)
        assert cache.working_lens.cpu().tolist() == lens
        _same_bits(cache.working_key.cpu(), work_k)
        _same_bits(cache.working_value.cpu(), work_v)


@pytest.mark.parametrize("seed", range(24))
def test_random_rows_positions_and_groups(cuda, seed):
    """Seeded random batches: rows on permuted spare slots at random positions (0 to the
    last cache row), GQA groups 1-32, head_dim 64/128/256, budgets 64-2048, bf16/fp16,
    output padding rows; one step with host positions, one reading the working lengths."""
    import random

    rnd = random.Random(500 + seed)
    hkv = rnd.choice([1, 2, 4, 8])
    group = rnd.choice([1, 2, 4, 8, 16, 32])
    dim = rnd.choice([64, 128, 256])
    budget = rnd.choice([64, 512, 2048])
    dtype = rnd.choice([torch.bfloat16, torch.float16])
    num_slots = rnd.randint(1, 24)
    rows = rnd.randint(1, num_slots)
    slots = rnd.sample(range(num_slots), rows)
    lengths = [rnd.choice([0, budget - 2, rnd.randint(0, budget - 2)]) for _ in range(rows)]
    print(f"seed {seed}: {rows} rows of {num_slots} slots, {hkv * group}/{hkv} heads x {dim}, budget {budget}, "
          f"{dtype}, lengths {lengths}", flush=True)
    case = Case(900 + seed, num_slots, hkv, hkv * group, dim, budget, dtype)
    for s, n in zip(slots, lengths):
        case.fill(s, n)
    tokens = rows + rnd.choice([0, 3])
    dev = Device(case, cuda, tokens)
    _step(case, dev, cuda, slots, lengths, tokens, dim ** -0.5)
    _step(case, dev, cuda, slots, None, tokens, dim ** -0.5)
