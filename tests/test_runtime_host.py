"""Host logic of DiffSpecDraftCache on the CPU, with the launch chain replaced by a recorder.

Mirrors the reference's runtime tests, which replace the score kernel by
attribute (tests/test_runtime.py:127, :566-579): slot stability across
reorder and cancellation (tests/test_runtime.py:755-778), the retrieval
skip rules and counters (tests/test_runtime.py:532-612), the verifier rows
handed to the device (committed query, rejected-suffix cut, graph padding;
diffspec/runtime.py:1211-1276), the LSE orientations
(diffspec/runtime.py:880-894) and the compact-prefill rebuild
(diffspec/runtime.py:1737-1765).  No GPU is used: every launch is recorded.
"""

from dataclasses import dataclass
from types import SimpleNamespace

import pytest
import torch

from ds355 import runtime, step


class _Rotary:
    rotary_dim = 2
    is_neox_style = True

    def __init__(self, positions=64):
        self.cos_sin_cache = torch.zeros((positions, 2))


@dataclass(frozen=True)
class _ReferenceShapedSettings:
    """The reference proposer's settings type: exactly the 7 fields of diffspec/runtime.py:18-27, no recent_window."""

    chunk_size: int
    token_budget: int
    retrieval_interval: int
    max_tree_nodes: int
    max_tree_depth: int
    tree_threshold: float
    adaptive_profile: bool


def _cache(settings_type=runtime.DiffSpecSettings, **overrides):
    settings = dict(chunk_size=2, token_budget=8, retrieval_interval=2, max_tree_nodes=4, max_tree_depth=2,
                    tree_threshold=0.7, adaptive_profile=False)
    settings.update(overrides.pop("settings", {}))
    kwargs = dict(max_num_reqs=4, max_model_len=16, num_kv_heads=1, head_dim=2, target_num_layers=2,
                  dtype=torch.float32, device=torch.device("cpu"), rotary_embedding=_Rotary())
    kwargs.update(overrides)
    return runtime.DiffSpecDraftCache(settings_type(**settings), **kwargs)


@pytest.fixture
def launches(monkeypatch):
    calls = []

    def record(**kw):
        calls.append({k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()})

    monkeypatch.setattr(step, "retrieval_step", record)
    return calls


def _first(t, n):
    """The first n entries of a per-row array (the runtime passes whole staging rows; kernels read batch_size)."""
    return t[:n].tolist()


def _metadata(query_ends, seq_lens, prefill):
    return SimpleNamespace(actual_seq_lengths_q=query_ends, seq_lens_list=seq_lens,
                           block_tables=torch.zeros((len(seq_lens), 1), dtype=torch.int32),
                           num_prefills=1 if prefill else 0)


def test_slots_stay_stable_across_reorder_and_cancellation():
    cache = _cache()
    cache.set_active_requests(["a", "b", "c"])
    slots = dict(cache._request_slots)
    assert sorted(slots.values()) == [0, 1, 2]
    cache.set_active_requests(["c", "a"])  # reorder + cancel "b"
    assert cache._request_slots == {"a": slots["a"], "c": slots["c"]}
    assert cache._active_slots == [slots["c"], slots["a"]]
    cache.sel_count[slots["b"]] = 5
    cache.set_active_requests(["c", "a", "d"])  # "d" takes the lowest free slot, b's
    assert cache._request_slots["d"] == slots["b"]
    with pytest.raises(RuntimeError, match="exhausted"):
        cache.set_active_requests(["a", "c", "d", "e", "f"])


def test_freed_slot_forgets_its_selection():
    cache = _cache()
    cache.set_active_requests(["a", "b"])
    cache.sel_count[:2] = 3
    cache.working_lens[:2] = 7
    cache.set_active_requests(["b"])
    freed = 0 if cache._request_slots["b"] == 1 else 1
    assert int(cache.sel_count[freed]) == -1 and int(cache.working_lens[freed]) == 0


def test_retrieval_skips_prefill_snapshot_and_interval(launches):
    cache = _cache()
    q = torch.arange(20, dtype=torch.float32).view(5, 2, 2)
    lse = torch.arange(10, dtype=torch.float32).view(5, 2, 1)
    key_cache = torch.zeros((1, 2, 1, 2))
    cache.begin_target_forward(["r0", "r1"])
    cache.capture_target_attention(q, lse, key_cache, _metadata([3, 5], [6, 4], prefill=True), 0.5)
    assert cache._target_query.shape == (2, 2, 2)  # the last query token of each prefill row
    torch.testing.assert_close(cache._target_query, q[[2, 4]])
    cache.accept_target_queries(torch.ones(2), is_prefill=True)
    assert launches == []
    cache.begin_target_forward(["r0", "r1"])
    cache.capture_target_attention(q[[2, 4]], lse[[2, 4]], key_cache, _metadata([1, 2], [6, 4], prefill=False), 0.5)
    cache.accept_target_queries(torch.ones(2), is_prefill=False)  # interval 2: first decode cycle skipped
    assert launches == []
    cache.accept_target_queries(torch.tensor([1, 1]), is_prefill=False)
    assert len(launches) == 1
    call = launches[0]
    assert call["stages"] == step.SCORE | step.SELECT  # 2 rows: the chain, so no rows moved at retrieval
    assert _first(call["rows"].counts, call["rows"].batch_size) == [1, 1]
    assert _first(call["rows"].query_start, call["rows"].batch_size) == [0, 1]
    assert _first(call["rows"].query_len, call["rows"].batch_size) == [1, 1]
    assert _first(call["rows"].target_len, call["rows"].batch_size) == [6, 4]
    assert call["slots"].tolist() == cache._active_slots
    assert call["snapshot"].scale == 0.5
    status = cache.retrieval_status()
    assert status["retrieval_skipped_prefill"] == 1
    assert status["retrieval_skipped_interval"] == 1
    assert status["retrieval_count"] == 1
    cache.begin_target_forward(["r1"])  # no capture: the previous snapshot must not be reused
    cache.accept_target_queries(torch.ones(1), is_prefill=cache.target_is_prefill)
    assert cache.retrieval_status()["retrieval_skipped_no_snapshot"] == 1
    assert len(launches) == 1


def test_slot_map_is_uploaded_only_when_it_changes():
    """Draft steps of one cycle reuse the device slot row; a new order re-uploads it."""
    cache = _cache()
    first = cache._device_slots([2, 0, 1])
    uploads = cache._slot_map.index
    again = cache._device_slots([2, 0, 1])
    assert cache._slot_map.index == uploads and again.data_ptr() == first.data_ptr()
    assert again.tolist() == [2, 0, 1]
    assert cache._device_slots([0, 1]).tolist() == [0, 1] and cache._slot_map.index != uploads


def test_snapshot_without_lse(launches):
    """A backend that returns no LSE: dropped as the reference does (runtime.py:850-851),
    or, with lse_free_scoring, kept and scored with per-row LSE buffers."""
    q = torch.zeros((2, 2, 2))
    meta = _metadata([1, 2], [6, 4], prefill=False)
    reference = _cache(settings=dict(retrieval_interval=1))
    reference.begin_target_forward(["a", "b"])
    reference.capture_target_attention(q, None, torch.zeros((1, 2, 1, 2)), meta, 0.5)
    reference.accept_target_queries(torch.ones(2), is_prefill=False)
    assert launches == [] and reference.retrieval_status()["retrieval_skipped_no_snapshot"] == 1

    cache = _cache(settings=dict(retrieval_interval=1), lse_free_scoring=True)
    cache.begin_target_forward(["a", "b"])
    cache.capture_target_attention(q, None, torch.zeros((1, 2, 1, 2)), meta, 0.5)
    cache.accept_target_queries(torch.ones(2), is_prefill=False)
    call = launches[-1]
    assert call["snapshot"].lse is None
    assert call["lse_partials"].shape == (2, cache.max_chunks, 2, 2)
    assert call["lse_out"].shape == (2, 2) and cache.scored_lse.shape == (cache.max_batch_rows, 2)
    # A supplied LSE is still used when there is one; no pair buffers are passed.
    cache.begin_target_forward(["a", "b"])
    cache.capture_target_attention(q, torch.ones((2, 2)), torch.zeros((1, 2, 1, 2)), meta, 0.5)
    cache.accept_target_queries(torch.ones(2), is_prefill=False)
    assert launches[-1]["snapshot"].lse is not None and launches[-1]["lse_partials"] is None


def test_speculative_rows_and_graph_padding(launches):
    """Linear verification: per-row query lengths, accepted counts and padded rows beyond the scheduler's."""
    cache = _cache(settings=dict(retrieval_interval=1), max_model_len=32)
    cache.begin_target_forward(["a", "b", "c"])
    q = torch.zeros((15, 2, 2))
    lse = torch.zeros((15, 2))
    # Three real rows of 5 query tokens; the capture holds two extra padded rows.
    meta = _metadata([5, 10, 15, 15, 15], [20, 30, 12, 1, 1], prefill=False)
    meta.block_tables = torch.zeros((5, 3), dtype=torch.int32)
    cache.capture_target_attention(q, lse, torch.zeros((4, 8, 1, 2)), meta, 1.0)
    cache.accept_target_queries(torch.tensor([3, 0, 5, 9, 9]), is_prefill=False)
    call = launches[-1]
    assert call["rows"].batch_size == 3  # padding rows are dropped (runtime.py:1211-1222)
    assert _first(call["rows"].counts, call["rows"].batch_size) == [3, 0, 5]
    assert _first(call["rows"].query_start, call["rows"].batch_size) == [0, 5, 10]
    assert _first(call["rows"].query_len, call["rows"].batch_size) == [5, 5, 5]
    assert _first(call["rows"].target_len, call["rows"].batch_size) == [20, 30, 12]
    assert call["score_partials"].shape == (3, cache.max_chunks, 1)
    # A verifier longer than the score buffer is refused on the host.
    meta.seq_lens_list = [40, 30, 12, 1, 1]
    cache.capture_target_attention(q, lse, torch.zeros((4, 8, 1, 2)), meta, 1.0)
    with pytest.raises(ValueError, match="exceeds the score buffer"):
        cache.accept_target_queries(torch.tensor([3, 0, 5, 9, 9]), is_prefill=False)


def test_lse_orientations_are_accepted():
    q = torch.zeros((3, 2, 4))
    flat = torch.arange(6.0)
    for lse in (flat, flat.view(3, 2), flat.view(3, 2).t().contiguous(), flat.view(3, 2, 1)):
        got = runtime.DiffSpecDraftCache._reshape_target_lse(q, lse)
        assert got.shape == (3, 2)
    transposed = runtime.DiffSpecDraftCache._reshape_target_lse(q, flat.view(3, 2).t().contiguous())
    torch.testing.assert_close(transposed, flat.view(3, 2))
    with pytest.raises(ValueError, match="does not match"):
        runtime.DiffSpecDraftCache._reshape_target_lse(q, torch.zeros(7))


def test_compact_prefill_launches_the_plan_stage(launches):
    cache = _cache(settings=dict(recent_window=4))
    cache.set_active_requests(["a", "b"])
    out = cache.prepare_compact_prefill(None, 2, committed_seq_lens=[9, 5])
    call = launches[-1]
    assert call["stages"] == step.PLAN
    assert call["slots"].tolist() == cache._active_slots
    assert call["committed_lens"].tolist() == [9, 5]
    assert call["recent_window"] == 4
    assert call["history_budget"] == 4  # ((8 - 2 - 1) // 2) * 2
    assert call["chunk_size"] == 2 and call["rotary_dim"] == 2 and call["is_neox_style"]
    assert out.shape == (2,)
    with pytest.raises(RuntimeError, match="omit active request rows"):
        cache.prepare_compact_prefill(None, 3, committed_seq_lens=[9, 5, 1])


def test_compact_prefill_reads_committed_lengths_from_device_tensor(launches):
    cache = _cache()
    cache.set_active_requests(["a"])
    cache.prepare_compact_prefill(None, 1, committed_seq_lens=torch.tensor([7], dtype=torch.int32))
    assert launches[-1]["committed_lens"].tolist() == [7]
    assert launches[-1]["recent_window"] == 2  # default: one chunk, the reference's tail


def test_tensor_parallel_scoring_is_refused(launches):
    cache = _cache(settings=dict(retrieval_interval=1), target_tensor_parallel_size=2)
    cache.begin_target_forward(["a"])
    cache.capture_target_attention(torch.zeros((1, 2, 2)), torch.zeros((1, 2)), torch.zeros((1, 4, 1, 2)),
                                   _metadata([1], [4], prefill=False), 1.0)
    with pytest.raises(NotImplementedError, match="all-reduce"):
        cache.accept_target_queries(torch.ones(1), is_prefill=False)
    with pytest.raises(ValueError, match="positive"):
        _cache(target_tensor_parallel_size=0)


@pytest.fixture
def attention_calls(monkeypatch):
    from ds355 import attention

    calls = []

    def record(query, key, value, output, working_key, working_value, working_lens, slots, positions=None, *,
               scale, workspace, reuse=None, reuse_key=None):
        calls.append(dict(slots=slots.tolist() if isinstance(slots, torch.Tensor) else list(slots),
                          positions=positions.tolist() if isinstance(positions, torch.Tensor) else positions,
                          scale=scale, rows=output.shape[0]))
        return output

    monkeypatch.setattr(attention, "draft_linear_attention", record)
    monkeypatch.setattr(attention, "attention_workspace_bytes", lambda *a: 64)
    monkeypatch.setattr(attention, "new_attention_workspace",
                        lambda *a: torch.zeros(64, dtype=torch.uint8))
    return calls


def test_draft_attention_pending_state(launches, attention_calls):
    """Compact prefill arms the root step at the slots' working lengths
    (runtime.py:1366-1369); later steps re-arm (runtime.py:1862-1871); the
    pending state is consumed by one forward_attention (runtime.py:2075-2076)."""
    cache = _cache()
    q = torch.zeros((3, 2, 2))
    kv = torch.zeros((3, 1, 2))
    with pytest.raises(RuntimeError, match="called without prepared state"):
        cache.forward_attention(q, kv, kv, 0.5, torch.zeros_like(q))
    cache.set_active_requests(["a", "b"])
    cache.set_active_requests(["b", "c"])  # slots 1, 0 after the reorder
    cache.prepare_compact_prefill(None, 2, committed_seq_lens=[9, 5])
    assert cache.has_pending_attention()
    cache.forward_attention(q, kv, kv, 0.5, torch.zeros_like(q))
    assert attention_calls[-1] == dict(slots=[1, 0], positions=None, scale=0.5, rows=3)
    assert not cache.has_pending_attention()
    cache.prepare_draft_step()
    cache.forward_attention(q, kv, kv, 0.25, torch.zeros_like(q))
    assert attention_calls[-1]["slots"] == [1, 0] and attention_calls[-1]["positions"] is None
    cache._pending_request_indices = [0, 1]
    cache._pending_local_positions = [3, 7]
    cache.forward_attention(q, kv, kv, 0.25, torch.zeros_like(q))
    assert attention_calls[-1]["slots"] == [0, 1] and attention_calls[-1]["positions"] == [3, 7]
    cache._pending_request_indices = [0]
    cache._pending_local_positions = [8]
    with pytest.raises(RuntimeError, match="DiffSpec working cache exhausted"):
        cache.forward_attention(q, kv, kv, 0.25, torch.zeros_like(q))


@pytest.fixture
def capture_calls(monkeypatch):
    from ds355 import capture

    calls = []

    def record(key, value, raw_key, raw_value, token_slots, absolute_positions, rope_buffer, *, tokens,
               working_lens=None, local_positions=None, prev_count=0, status=None, reuse=None,
               reuse_key=None):
        calls.append(dict(slots=token_slots[:tokens].tolist(), positions=absolute_positions.reshape(-1).tolist(),
                          tokens=tokens, rope=rope_buffer is not None, working_lens=working_lens is not None,
                          key=key[:tokens].clone()))
        if rope_buffer is None:
            return None
        count = absolute_positions.numel()
        return rope_buffer[:count].view(absolute_positions.shape)

    monkeypatch.setattr(capture, "capture_raw_kv_rows", record)
    return calls


@pytest.mark.parametrize("settings_type", [runtime.DiffSpecSettings, _ReferenceShapedSettings],
                         ids=["ds355-settings", "reference-7-field-settings"])
def test_linear_call_sequence_of_the_plugin(launches, attention_calls, capture_calls, settings_type):
    """The hooks the unchanged plugin calls on one linear verify + draft cycle, in its order:
    the runner's prepare_target_batch (ascend_patch.py:274) and begin_target_forward (:301),
    the attention patch's is_target_retrieval_layer / capture_target_attention (:198, :233)
    and target_tree_active reads (:165, :279, :311), the proposer's clear_proposed_tree
    (proposer.py:357), accept_target_queries (:216), prepare_inputs_padded's
    target_tree_active read (:224), begin_cycle (:103), populate_prefill (:266),
    prepare_compact_prefill (:303), the draft layer's capture + attention, end_cycle (:119)."""
    cache = _cache(settings_type, settings=dict(retrieval_interval=1, token_budget=16), max_model_len=32,
                   target_num_layers=3)
    assert cache.recent_window == 2  # the reference's settings carry no window: one chunk
    ids = ["a", "b"]
    # Verifier step: the runner activates the batch (linear: no proposed tree).
    cache.prepare_target_batch(ids, {"a": [5, 6, 7], "b": [1, 2, 3]})
    assert cache.target_tree_active is False
    cache.begin_target_forward(ids)
    assert cache._active_slots == [0, 1]
    assert [cache.is_target_retrieval_layer(i) for i in range(3)] == [False, False, True]
    assert not cache.has_pending_attention()  # the target's attention is not diverted
    q = torch.zeros((8, 2, 2))
    lse = torch.zeros((8, 2))
    meta = _metadata([4, 8], [20, 12], prefill=False)
    cache.capture_target_attention(q, lse, torch.zeros((4, 8, 1, 2)), meta, 0.5)
    assert cache.target_tree_active is False  # the sampler keeps its own path
    # Proposer: linear proposal, retrieval on the accepted counts.
    cache.clear_proposed_tree()
    assert cache.proposed_token_ids is None and cache.proposed_depths_cpu == []
    cache.accept_target_queries(torch.tensor([2, 4]), is_prefill=cache.target_is_prefill)
    assert launches[-1]["stages"] == step.SCORE | step.SELECT
    assert _first(launches[-1]["rows"].counts, 2) == [2, 4]
    assert not cache.target_tree_active  # prepare_inputs_padded returns its result unchanged
    with pytest.raises(RuntimeError, match="tree has not been verified"):
        cache.accepted_target_token_indices()
    cache.rewrite_target_positions([0, 1, 2], [3])  # no-op in linear verification
    # Draft cycle: project the padded prefill's raw K/V, then rebuild at the committed roots.
    cache.begin_cycle(ids)
    positions = torch.tensor([16, 17, 18, 19, 8, 9, 10, 11], dtype=torch.int64)
    raw_kv = torch.arange(16, dtype=torch.float32).view(8, 2)
    cache.populate_prefill(positions, raw_kv, raw_kv, meta)
    scatter = capture_calls[-1]
    assert scatter["slots"] == [0, 0, 0, 0, 1, 1, 1, 1]  # token -> row from the query ends -> slot
    assert scatter["positions"] == positions.tolist() and scatter["tokens"] == 8
    assert not scatter["rope"] and not scatter["working_lens"]  # raw rows only (runtime.py:1336-1347)
    torch.testing.assert_close(scatter["key"], raw_kv)
    cache.prepare_compact_prefill(meta, 2, committed_seq_lens=[18, 12])
    assert launches[-1]["stages"] == step.PLAN and launches[-1]["committed_lens"].tolist() == [18, 12]
    assert cache.has_pending_attention()
    # The draft layer: capture (the vllm::diffspec_capture_raw_kv op body) then attention.
    roots = torch.tensor([17, 11], dtype=torch.int64)
    rope = cache.graph_safe_rope_positions(roots, cache.capture_raw_kv(0, roots, raw_kv[:2], raw_kv[:2]))
    assert capture_calls[-1]["slots"] == [0, 1] and capture_calls[-1]["working_lens"]
    assert rope.shape == roots.shape
    cache.forward_attention(torch.zeros((2, 2, 2)), raw_kv[:2].view(2, 1, 2), raw_kv[:2].view(2, 1, 2), 0.5,
                            torch.zeros((2, 2, 2)))
    assert attention_calls[-1]["slots"] == [0, 1]
    cache.end_cycle()
    assert not cache.has_pending_attention()
    # Outside a cycle populate_prefill still maps tokens by the query ends; an empty call is a no-op.
    cache.populate_prefill(positions[:0], raw_kv[:0], raw_kv[:0], meta)
    assert len(capture_calls) == 2


def test_retrieval_with_host_counts_and_no_committed_rows_is_skipped(launches):
    """All-zero host counts: skipped and counted, as runtime.py:1253-1257 does."""
    cache = _cache(settings=dict(retrieval_interval=1))
    cache.begin_target_forward(["a", "b"])
    cache.capture_target_attention(torch.zeros((2, 2, 2)), torch.zeros((2, 2)), torch.zeros((1, 2, 1, 2)),
                                   _metadata([1, 2], [6, 4], prefill=False), 0.5)
    cache.accept_target_queries(torch.tensor([0, 0]), is_prefill=False)
    assert launches == []
    status = cache.retrieval_status()
    assert status["retrieval_skipped_no_committed_tokens"] == 1 and status["retrieval_count"] == 0
    cache.accept_target_queries(torch.tensor([0, 1]), is_prefill=False)
    assert len(launches) == 1 and cache.retrieval_status()["retrieval_count"] == 1


def test_cached_step_descriptors_follow_the_partial_buffers(monkeypatch):
    """A validated descriptor is reused for its layout, and dropped when the buffers it points to are replaced."""
    built, launched = [], []

    def record(**kw):
        built.append(kw["score_partials"].data_ptr())
        desc = SimpleNamespace(partials=kw["score_partials"].data_ptr())
        kw["reuse"][kw["reuse_key"]] = (desc, torch.device("cpu"))

    monkeypatch.setattr(step, "retrieval_step", record)
    monkeypatch.setattr(step, "launch", lambda desc, device, stages=None: launched.append(desc))
    cache = _cache(settings=dict(retrieval_interval=1))
    q = torch.ones((2, 2, 2))
    lse = torch.zeros((2, 2))

    def retrieve(kv_heads, counts):
        cache.begin_target_forward(["r0", "r1"])
        cache.capture_target_attention(q, lse, torch.zeros((1, 2, kv_heads, 2)), _metadata([1, 2], [6, 4], False), 0.5)
        cache.accept_target_queries(counts, is_prefill=False)

    retrieve(1, torch.tensor([1, 1], dtype=torch.int32))
    retrieve(1, torch.tensor([1, 2], dtype=torch.int32))  # same layout: the cached descriptor, refreshed
    assert len(built) == 1 and len(launched) == 1
    assert launched[0].counts != 0 and launched[0].scale == 0.5
    assert launched[0].query == cache._target_query.data_ptr()
    retrieve(2, torch.tensor([1, 1], dtype=torch.int32))  # two KV heads: new partial buffer, new descriptor
    retrieve(1, torch.tensor([1, 1], dtype=torch.int32))  # back to one head: rebuilt, not the stale descriptor
    assert len(built) == 3 and len(launched) == 1
    assert built[2] == cache._score_partials.data_ptr()


def test_rows_staged_with_the_snapshot_follow_the_active_slots(monkeypatch):
    """Rows uploaded when the snapshot is taken are used unless the active slots changed since."""
    seen = []

    def record(**kw):
        seen.append(("built", kw["rows"].query_start[:2].tolist(), kw["rows"].query_len[:2].tolist(),
                     kw["rows"].target_len[:2].tolist(), kw["slots"][:2].tolist()))
        kw["reuse"][kw["reuse_key"]] = (SimpleNamespace(), torch.device("cpu"))

    def launch(desc, device, stages=None):
        rows = cache._rows_staging.device
        seen.append(("launched", rows[0, :2].tolist(), rows[1, :2].tolist(), rows[2, :2].tolist(),
                     rows[3, :2].tolist()))

    monkeypatch.setattr(step, "retrieval_step", record)
    monkeypatch.setattr(step, "launch", launch)
    cache = _cache(settings=dict(retrieval_interval=1))
    q, lse, kc = torch.ones((3, 2, 2)), torch.zeros((3, 2)), torch.zeros((1, 2, 1, 2))
    cache.begin_target_forward(["a", "b"])
    cache.capture_target_attention(q, lse, kc, _metadata([1, 3], [6, 4], False), 0.5)
    cache.accept_target_queries(torch.tensor([1, 2], dtype=torch.int32), is_prefill=False)
    slots_ab = list(cache._active_slots)
    assert seen[-1] == ("built", [0, 1], [1, 2], [6, 4], slots_ab)
    cache.begin_target_forward(["a", "b"])
    cache.capture_target_attention(q, lse, kc, _metadata([2, 3], [9, 5], False), 0.5)
    cache.accept_target_queries(torch.tensor([1, 1], dtype=torch.int32), is_prefill=False)
    assert seen[-1] == ("launched", [0, 2], [2, 1], [9, 5], slots_ab)
    cache.begin_target_forward(["a", "b"])
    cache.capture_target_attention(q, lse, kc, _metadata([1, 2], [7, 8], False), 0.5)
    cache.set_active_requests(["b", "a"])  # reordered after the snapshot: the rows are staged again
    cache.accept_target_queries(torch.tensor([1, 1], dtype=torch.int32), is_prefill=False)
    assert seen[-1] == ("launched", [0, 1], [1, 1], [7, 8], slots_ab[::-1])


def test_gather_records_follow_the_slot_map(launches):
    """A request leaving its slot changes that slot's selection generation (its
    gather records describe the request that left); slots that keep their
    request keep theirs.  Every rebuild passes the cache's records, and the
    retrieval call moves the final history rows when it runs as the single launch (prefix_at_retrieval)."""
    cache = _cache()
    cache.set_active_requests(["a", "b", "c"])
    assert cache.sel_gen.tolist() == [0, 0, 0, 0]
    cache.sel_gen[:] = torch.tensor([5, 6, 7, 0], dtype=torch.int32)
    cache.set_active_requests(["c", "a"])  # b leaves slot 1
    assert cache.sel_gen.tolist() == [5, 7, 7, 0]
    assert cache.sel_count[1].item() == -1
    cache.set_active_requests(["c", "a", "d"])  # d takes the freed slot with a new generation
    assert cache._request_slots["d"] == 1 and cache.sel_gen.tolist() == [5, 7, 7, 0]
    cache.prepare_compact_prefill(None, 3, committed_seq_lens=[9, 9, 9])
    gen, records = launches[-1]["gather_records"]
    assert launches[-1]["stages"] == step.PLAN
    assert gen.tolist() == cache.sel_gen.tolist() and records.shape == cache.gather_records.shape
    assert runtime.RETRIEVAL_STAGES == step.SCORE | step.SELECT
    # By default the final history rows move at retrieval exactly when it runs as the single launch.
    assert cache.retrieval_stages_for(8) == step.SCORE | step.SELECT | step.PREFIX
    assert cache.retrieval_stages_for(7) == step.SCORE | step.SELECT
    assert _cache(prefix_at_retrieval=False).retrieval_stages_for(16) == step.SCORE | step.SELECT
    assert _cache(prefix_at_retrieval=True).retrieval_stages_for(1) == step.SCORE | step.SELECT | step.PREFIX


def _speculative_config(**overrides):
    fields = dict(diffspec_chunk_size=32, diffspec_token_budget=2048, diffspec_retrieval_interval=4,
                  diffspec_max_tree_nodes=50, num_speculative_tokens=4, diffspec_tree_threshold=0.7,
                  diffspec_adaptive_profile=False, enabled=True)
    fields.update(overrides)
    spec = SimpleNamespace(**fields)
    spec.use_diffspec = lambda: spec.enabled
    return SimpleNamespace(speculative_config=spec)


def test_settings_from_vllm_config_follow_the_reference_mapping():
    """diffspec/runtime.py:28-41: max_tree_depth comes from num_speculative_tokens; a disabled policy raises."""
    settings = runtime.DiffSpecSettings.from_vllm_config(_speculative_config())
    assert settings == runtime.DiffSpecSettings(chunk_size=32, token_budget=2048, retrieval_interval=4,
                                                max_tree_nodes=50, max_tree_depth=4, tree_threshold=0.7,
                                                adaptive_profile=False, recent_window=None)
    windowed = runtime.DiffSpecSettings.from_vllm_config(_speculative_config(diffspec_recent_window=256))
    assert windowed.recent_window == 256
    with pytest.raises(ValueError, match="enabled DiffSpec policy"):
        runtime.DiffSpecSettings.from_vllm_config(_speculative_config(enabled=False))
    with pytest.raises(ValueError, match="enabled DiffSpec policy"):
        runtime.DiffSpecSettings.from_vllm_config(SimpleNamespace(speculative_config=None))
    cache = _cache(settings=dict(chunk_size=2, token_budget=8), recent_window=6)
    assert cache.recent_window == 6  # the constructor argument wins over the settings


def test_reference_settings_construct_the_cache_with_the_proposer_arguments():
    """The proposer's constructor call (proposer.py:52-65) on the reference's 7-field settings."""
    settings = _ReferenceShapedSettings(chunk_size=2, token_budget=8, retrieval_interval=4, max_tree_nodes=4,
                                        max_tree_depth=2, tree_threshold=0.7, adaptive_profile=True)
    cache = runtime.DiffSpecDraftCache(
        settings, max_num_reqs=4, max_model_len=16, num_kv_heads=1, head_dim=2, target_num_layers=2,
        dtype=torch.float32, device=torch.device("cpu"), rotary_embedding=_Rotary(), target_cos_sin_cache=None,
        target_tensor_parallel_size=1)
    assert cache.history_budget == 4 and cache.recent_window == 2
    assert cache.retrieval_interval == 4 and cache.controller.adaptive
    assert cache.controller.profile == runtime.DiffSpecTreeProfile(50, 10)  # proposer.py:411 reads it
    with pytest.raises(ValueError, match="too small for tree tokens"):
        runtime.DiffSpecDraftCache(
            _ReferenceShapedSettings(2, 3, 4, 4, 2, 0.7, False), max_num_reqs=4, max_model_len=16, num_kv_heads=1,
            head_dim=2, target_num_layers=2, dtype=torch.float32, device=torch.device("cpu"),
            rotary_embedding=_Rotary())


class _SelectingRecorder:
    """Stands in for the step: each scored row (count > 0) stores the selection the test scripted for its slot."""

    def __init__(self):
        self.next = {}
        self.calls = 0

    def __call__(self, **kw):
        self.calls += 1
        counts = kw["rows"].counts[: kw["rows"].batch_size].tolist()
        for row, slot in enumerate(kw["slots"].tolist()):
            if counts[row] > 0 and slot in self.next:
                ids = self.next[slot]
                kw["sel_ids"][slot, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
                kw["sel_count"][slot] = len(ids)


def _verify(cache, counts, lens=(20, 12)):
    cache.begin_target_forward(["a", "b"])
    cache.capture_target_attention(torch.zeros((2, 2, 2)), torch.zeros((2, 2)), torch.zeros((4, 8, 1, 2)),
                                   _metadata([1, 2], list(lens), prefill=False), 0.5)
    cache.accept_target_queries(torch.tensor(counts), is_prefill=False)


def test_adaptive_cadence_doubles_on_stable_selections(monkeypatch):
    """runtime.py:575-593 fed at :1309-1331: intersection over union >= 0.9 and no acceptance drop double the
    interval (capped at 32); a changed selection or a >10% acceptance drop returns it to the base."""
    recorder = _SelectingRecorder()
    monkeypatch.setattr(step, "retrieval_step", recorder)
    cache = _cache(settings=dict(retrieval_interval=1, adaptive_profile=True, token_budget=16), max_model_len=32)
    slot_a = 0
    expected_calls = 0

    def cycle(counts, selection_a, interval_after):
        nonlocal expected_calls
        recorder.next = {slot_a: selection_a, 1: [9]}
        before = recorder.calls
        _verify(cache, counts)
        if recorder.calls > before:
            expected_calls += 1
        # The observation is applied at the next call, before the interval is read.
        cache._observe_previous_retrieval()
        assert cache.retrieval_interval == interval_after

    cycle([3, 1], [0, 1, 2], 1)  # cycle 1: first selection, no previous chunks, overlap 0 -> base
    cycle([3, 1], [0, 1, 2], 2)  # cycle 2: same chunks, same acceptance (2) -> doubled
    cycle([3, 1], [0, 1, 3], 2)  # cycle 3: 3 % 2, skipped: nothing observed, whatever the scores
    cycle([3, 1], [0, 1, 2], 4)  # cycle 4 retrieves: doubled again
    for _ in range(3):
        cycle([3, 1], [0, 1, 2], 4)  # cycles 5-7 skipped
    cycle([3, 1], [0, 1, 3], 1)  # cycle 8: overlap 2/4 -> base
    cycle([3, 1], [0, 1, 3], 2)  # cycle 9: stable -> 2
    cycle([2, 1], [0, 1, 3], 1)  # cycle 10: acceptance 1 < 0.9 * 2 -> base, though stable
    cycle([2, 1], [0, 1, 3], 2)  # cycle 11: acceptance 1 again -> 2
    # Cycle 12: row 0 committed nothing, so the first scored row is row 1 (slot 1, selection [9] before and
    # after: stable), with acceptance 0 < 0.9 * 1 -> base.
    cycle([0, 1], [5], 1)
    assert cache._adaptive_ids[1, slot_a, :3].tolist() == [0, 1, 3]  # row 0 kept its selection
    cycle([2, 1], [0, 1, 3], 2)  # cycle 13
    cycle([2, 1], [0, 1, 3], 4)  # cycle 14
    cycle([2, 1], [0, 1, 3], 4)  # 15 skipped
    cycle([2, 1], [0, 1, 3], 8)  # 16
    for _ in range(7):
        cycle([2, 1], [0, 1, 3], 8)  # 17-23 skipped
    cycle([2, 1], [0, 1, 3], 16)  # 24
    for _ in range(7):
        cycle([2, 1], [0, 1, 3], 16)  # 25-31 skipped
    cycle([2, 1], [0, 1, 3], 32)  # 32
    for _ in range(31):
        cycle([2, 1], [0, 1, 3], 32)  # 33-63 skipped
    cycle([2, 1], [0, 1, 3], 32)  # 64: capped at 32
    assert expected_calls == recorder.calls == 14  # cycles 1, 2, 4, 8-14, 16, 24, 32 and 64
    status = cache.retrieval_status()
    assert status["retrieval_count"] == 14 and status["retrieval_skipped_interval"] == 64 - 14


def test_adaptive_cadence_off_keeps_the_interval(monkeypatch):
    """adaptive_profile=False: the base interval always, and no host copies are made."""
    recorder = _SelectingRecorder()
    monkeypatch.setattr(step, "retrieval_step", recorder)
    cache = _cache(settings=dict(retrieval_interval=2, token_budget=16), max_model_len=32)
    for _ in range(8):
        recorder.next = {0: [0, 1, 2], 1: [9]}
        _verify(cache, [3, 1])
        assert cache.retrieval_interval == 2 and cache._adaptive_pending is None
    assert recorder.calls == 4
