"""GPU: raw pre-RoPE K/V capture and the graph-safe RoPE input against the oracle.

Mirrors the reference's graph-replay tests (tests/test_kv_graph_replay.py:19-108):
every draft step writes its token's pre-RoPE K/V at the absolute position, the
cache-owned RoPE input keeps its address and carries the local position
(4, 5, 6 for a root rebuilt at history length 4), graph padding is neither
written nor given a position, and stale positions of a larger previous call
are zeroed.  Raw caches are compared bit for bit with the oracle's
``write_raw``; RoPE buffers exactly with its ``graph_safe_rope_positions``.
"""

from types import SimpleNamespace

import pytest
import torch

from helpers import assert_attention_close, attention_terms, gen, randn
from oracle import diffspec_oracle as O

pytestmark = pytest.mark.gpu


class _Rotary:
    def __init__(self, rotary_dim, rows, dtype):
        self.rotary_dim = rotary_dim
        self.is_neox_style = True
        self.cos_sin_cache = O.rope_cos_sin_cache(max(rotary_dim, 2), rows, 1.0e6).to(dtype)


def _cache(cuda, *, head_dim, dtype, max_num_reqs=1, max_model_len=12, kv_heads=1, settings=(2, 8, 8, 4, 3, 0.7, False),
           rotary_dim=0):
    from ds355 import runtime

    return runtime.DiffSpecDraftCache(
        runtime.DiffSpecSettings(*settings), max_num_reqs=max_num_reqs, max_model_len=max_model_len,
        num_kv_heads=kv_heads, head_dim=head_dim, target_num_layers=2, dtype=dtype, device=cuda,
        rotary_embedding=_Rotary(rotary_dim, max(settings[1], 16), dtype))


@pytest.mark.parametrize("padding", [0, 3])
@pytest.mark.parametrize("prepared_root", [False, True])
def test_capture_updates_each_draft_step_and_local_position(cuda, padding, prepared_root):
    """tests/test_kv_graph_replay.py:19-87 at head_dim 64 (the attention kernel's smallest):
    positions 5, 6, 7 of one request with a 6-token committed context; chunk 2, budget 8,
    depth 3 give history 4, so the local positions are 4, 5, 6."""
    cache = _cache(cuda, head_dim=64, dtype=torch.bfloat16)
    cache.begin_cycle(["request-0"])
    cache.raw_key.zero_()
    cache.raw_value.zero_()
    metadata = SimpleNamespace(actual_seq_lengths_q=[1], seq_lens_list=[6])
    if prepared_root:
        cache.prepare_compact_prefill(metadata, 1)
    captured = None
    observed = []
    for step in range(3):
        key = torch.full((1 + padding, 64), 999.0, dtype=torch.bfloat16, device=cuda)
        key[0] = torch.arange(64, device=cuda) * 0.125 + step
        value = key + 10
        positions = torch.full((1 + padding,), 11, dtype=torch.int32, device=cuda)
        positions[0] = 5 + step
        result = cache.capture_raw_kv(0, positions, key, value, metadata)
        result = cache.graph_safe_rope_positions(positions, result)
        if captured is None:
            captured = result
        assert result.data_ptr() == captured.data_ptr()
        assert result.shape == positions.shape
        assert result.cpu().tolist() == [4 + step] + [0] * padding
        observed.append(int(result[0]))
        assert cache.has_pending_attention()
        assert torch.equal(cache.raw_key[0, 5 + step, 0], key[0])
        assert torch.equal(cache.raw_value[0, 5 + step, 0], value[0])
        output = torch.full((1 + padding, 1, 64), float("nan"), dtype=torch.bfloat16, device=cuda)
        cache.forward_attention(torch.ones((1 + padding, 1, 64), dtype=torch.bfloat16, device=cuda),
                                key.view(1 + padding, 1, 64), value.view(1 + padding, 1, 64), 1.0, output)
        assert torch.isfinite(output[:1]).all()
        assert output[1:].count_nonzero() == 0
        assert not cache.has_pending_attention()
    assert observed == [4, 5, 6]
    assert cache._draft_step == 3 + int(prepared_root)
    assert cache.raw_key[0, 11].count_nonzero() == 0
    assert cache.capture_status() == 0


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_rope_buffer_keeps_address_and_zeroes_stale_tail(cuda, dtype):
    """tests/test_kv_graph_replay.py:89-108 on the device buffer, step by step against the oracle."""
    cache = _cache(cuda, head_dim=2, dtype=torch.float32)
    absolute = torch.tensor([7, 8, 9, 10], dtype=dtype, device=cuda)
    captured = cache.graph_safe_rope_positions(absolute, None)
    assert captured.cpu().tolist() == [7, 8, 9, 10]
    replay = cache.graph_safe_rope_positions(absolute[:1], torch.tensor([4], dtype=dtype, device=cuda))
    assert replay.data_ptr() == captured.data_ptr()
    assert captured.cpu().tolist() == [4, 0, 0, 0]
    cache.graph_safe_rope_positions(absolute, torch.tensor([5, 0, 0, 0], dtype=dtype, device=cuda))
    assert captured.cpu().tolist() == [5, 0, 0, 0]
    ref = torch.zeros(12, dtype=dtype)
    written = 4
    ref[:4] = torch.tensor([5, 0, 0, 0], dtype=dtype)
    for count in [8, 2, 7, 1, 0, 4]:
        positions = torch.arange(count, dtype=dtype)
        replay = cache.graph_safe_rope_positions(positions.to(cuda), positions.to(cuda))
        assert replay.untyped_storage().data_ptr() == captured.untyped_storage().data_ptr()
        _, written = O.graph_safe_rope_positions(ref, written, positions, positions)
        assert torch.equal(cache._rope_position_buffers[dtype].cpu(), ref)


@pytest.mark.parametrize("dtype,head_dim,heads", [(torch.bfloat16, 128, 4), (torch.float16, 64, 8),
                                                  (torch.float32, 2, 1), (torch.bfloat16, 96, 2),
                                                  (torch.float32, 128, 4)])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_capture_kernel_matches_oracle(cuda, dtype, head_dim, heads, index_dtype):
    """Strided K/V rows (views into a fused qkv projection), permuted slots, graph padding, the
    three RoPE modes and a stale tail, against write_raw / graph_safe_rope_positions."""
    from ds355.capture import capture_raw_kv_rows

    g = gen(head_dim * 10 + heads)
    slots_n, lmax, tokens, pad = 6, 64, 5, 3
    raw_k = randn((slots_n, lmax, heads, head_dim), dtype, g)
    raw_v = randn((slots_n, lmax, heads, head_dim), dtype, g)
    qkv = randn((tokens + pad, (4 + 2) * heads * head_dim), dtype, g)  # q of 4 x kv width, then k, v
    key = qkv[:, 4 * heads * head_dim: 5 * heads * head_dim]
    value = qkv[:, 5 * heads * head_dim:]
    slots = [4, 0, 5, 2, 1]
    positions = torch.tensor([63, 0, 17, 40, 5, 11, 11, 11], dtype=index_dtype)
    lens = torch.tensor([9, 3, 7, 30, 0, 12], dtype=torch.int32)
    exp_k, exp_v = raw_k.clone(), raw_v.clone()
    O.write_raw(exp_k, exp_v, slots, positions[:tokens].tolist(), key[:tokens], value[:tokens])

    d_k, d_v = raw_k.to(cuda), raw_v.to(cuda)
    d_qkv = qkv.to(cuda)
    d_key = d_qkv[:, 4 * heads * head_dim: 5 * heads * head_dim]
    d_value = d_qkv[:, 5 * heads * head_dim:]
    buffer = torch.full((16,), 77, dtype=index_dtype, device=cuda)
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    rope = capture_raw_kv_rows(d_key, d_value, d_k, d_v, torch.tensor(slots, dtype=torch.int32, device=cuda),
                               positions.to(cuda), buffer, tokens=tokens, working_lens=lens.to(cuda), prev_count=12,
                               status=status)
    torch.cuda.synchronize()
    assert torch.equal(d_k.cpu(), exp_k) and torch.equal(d_v.cpu(), exp_v)
    ref = torch.full((16,), 77, dtype=index_dtype)
    _, _ = O.graph_safe_rope_positions(ref, 12, positions, torch.tensor(
        [int(lens[s]) for s in slots] + [0] * pad, dtype=index_dtype))
    assert torch.equal(buffer.cpu(), ref)
    assert rope.cpu().tolist() == ref[:tokens + pad].tolist()
    assert int(status) == 0
    # absolute mode, shorter call: the tail of the previous call is cleared
    rope = capture_raw_kv_rows(d_key, d_value, d_k, d_v, torch.tensor(slots, dtype=torch.int32, device=cuda),
                               positions[:4].to(cuda), buffer, tokens=4, prev_count=8)
    torch.cuda.synchronize()
    O.graph_safe_rope_positions(ref, 8, positions[:4], None)
    assert torch.equal(buffer.cpu(), ref)


def test_out_of_range_token_is_skipped_and_flagged(cuda):
    from ds355.capture import capture_raw_kv_rows

    g = gen(3)
    raw_k = torch.zeros((2, 16, 1, 64), dtype=torch.bfloat16, device=cuda)
    raw_v = torch.zeros_like(raw_k)
    key = randn((3, 64), torch.bfloat16, g).to(cuda)
    positions = torch.tensor([3, 16, 5], dtype=torch.int64, device=cuda)  # 16 == max_model_len
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    buffer = torch.zeros(8, dtype=torch.int64, device=cuda)
    capture_raw_kv_rows(key, key, raw_k, raw_v, torch.tensor([1, 0, 2], dtype=torch.int32, device=cuda), positions,
                        buffer, tokens=3, status=status)  # slot 2 is out of range too
    torch.cuda.synchronize()
    assert int(status) & 1
    assert torch.equal(raw_k[1, 3, 0], key[0])
    assert raw_k.count_nonzero() == key[0].count_nonzero()
    assert buffer.cpu().tolist() == [3, 16, 5, 0, 0, 0, 0, 0]


def test_draft_cycle_capture_attention_against_oracle(cuda):
    """A reordered batch of 3 requests: retrieval rebuild, then three draft steps of
    capture + attention, every raw, working and output tensor against the oracle."""
    from ds355 import runtime

    heads, d, hq = 2, 128, 8
    settings = runtime.DiffSpecSettings(chunk_size=16, token_budget=256, retrieval_interval=1, max_tree_nodes=4,
                                        max_tree_depth=4, tree_threshold=0.7, adaptive_profile=False)
    cache = runtime.DiffSpecDraftCache(settings, max_num_reqs=4, max_model_len=512, num_kv_heads=heads, head_dim=d,
                                       target_num_layers=2, dtype=torch.bfloat16, device=cuda,
                                       rotary_embedding=_Rotary(d, 512, torch.bfloat16))
    g = gen(41)
    cache.raw_key.copy_(randn(cache.raw_key.shape, torch.bfloat16, g))
    cache.raw_value.copy_(randn(cache.raw_value.shape, torch.bfloat16, g))
    cache.working_key.fill_(float("nan"))
    cache.working_value.fill_(float("nan"))
    cache.set_active_requests(["a", "b", "c"])
    cache.begin_cycle(["c", "a", "b"])  # slots 2, 0, 1
    committed = [40, 300, 9]
    cache.prepare_compact_prefill(SimpleNamespace(seq_lens_list=committed), 3)
    torch.cuda.synchronize()
    raw_k, raw_v = cache.raw_key.cpu(), cache.raw_value.cpu()
    work_k, work_v = cache.working_key.cpu(), cache.working_value.cpu()
    lens = cache.working_lens.cpu().tolist()
    slots = list(cache._active_slots)
    for step in range(3):
        absolute = torch.tensor([c + step for c in committed] + [0], dtype=torch.int64)  # + one padding token
        key = randn((4, heads * d), torch.bfloat16, g)
        value = randn((4, heads * d), torch.bfloat16, g)
        q = randn((4, hq, d), torch.bfloat16, g)
        rope = cache.graph_safe_rope_positions(absolute.to(cuda), cache.capture_raw_kv(
            0, absolute.to(cuda), key.to(cuda), value.to(cuda), None))
        local = [lens[s] for s in slots]
        assert rope.cpu().tolist() == local + [0]
        O.write_raw(raw_k, raw_v, slots, absolute[:3].tolist(), key[:3], value[:3])
        # vLLM would rotate q and k at `rope`; the identity keeps the check on this path's data
        out = torch.full((4, hq, d), float("nan"), dtype=torch.bfloat16, device=cuda)
        cache.forward_attention(q.to(cuda), key.view(4, heads, d).to(cuda), value.view(4, heads, d).to(cuda),
                                d ** -0.5, out)
        expected = torch.empty_like(q)
        O.draft_linear_attention(q, key.view(4, heads, d), value.view(4, heads, d), d ** -0.5, expected, work_k,
                                 work_v, lens, slots, local)
        torch.cuda.synchronize()
        terms = torch.zeros((4, hq, d))
        terms[: len(slots)] = attention_terms(q[: len(slots)], work_k, work_v, slots, local, d ** -0.5)
        assert_attention_close(out.cpu(), expected, terms)
        assert torch.equal(cache.raw_key.cpu(), raw_k) and torch.equal(cache.raw_value.cpu(), raw_v)
        assert cache.working_lens.cpu().tolist() == lens
    cache.end_cycle()
    assert cache.capture_status() == 0
