"""GPU: the launches replayed from a HIP graph give the eager results.

The plugin's draft model runs under graph capture: every draft step replays
the same kernel nodes on the same buffers while the host rewrites their
contents in place (diffspec/runtime.py:1767-1794 keeps the RoPE input at one
address for exactly that; tests/test_kv_graph_replay.py:19-108 checks it on
a compiled graph).  Here the real HIP graph of each launch sequence is
captured once and replayed several times, with eager work and
synchronisation between the replays; after every replay the state is
compared bit for bit with the same launches run eagerly on the same inputs.
The launches hold no host-side state that a replay would freeze: positions,
working lengths, slots and the workspaces' epochs are read on the device.
"""

import pytest
import torch

from helpers import assert_attention_close, attention_terms, gen, randn
from oracle import diffspec_oracle as O
from test_gpu_step import build_case, check_step

pytestmark = pytest.mark.gpu


def _same(a, b, name):
    assert torch.equal(a.isnan(), b.isnan()), name
    assert torch.equal(torch.nan_to_num(a), torch.nan_to_num(b)), name


def test_draft_steps_replayed_from_a_graph(cuda):
    """Raw-KV capture + draft attention, captured once and replayed as three draft steps."""
    from ds355 import attention, capture

    g = gen(41)
    num_slots, hkv, hq, d, budget, lmax = 4, 2, 8, 128, 512, 600
    dt = torch.bfloat16
    slots = torch.tensor([2, 0, 3], dtype=torch.int32, device=cuda)
    rows = slots.numel()
    lens0 = torch.tensor([100, 7, 300, 64], dtype=torch.int32)
    work_k = torch.full((num_slots, hkv, budget, d), float("nan"), dtype=dt)
    work_v = work_k.clone()
    for s, n in enumerate(lens0.tolist()):
        work_k[s, :, :n] = randn((hkv, n, d), dt, g)
        work_v[s, :, :n] = randn((hkv, n, d), dt, g)

    def fresh():
        return dict(
            work_k=work_k.to(cuda), work_v=work_v.to(cuda), lens=lens0.to(cuda),
            raw_k=torch.zeros((num_slots, lmax, hkv, d), dtype=dt, device=cuda),
            raw_v=torch.zeros((num_slots, lmax, hkv, d), dtype=dt, device=cuda),
            rope=torch.zeros(8, dtype=torch.int64, device=cuda),
            out=torch.full((rows + 1, hq, d), float("nan"), dtype=dt, device=cuda),
            ws=attention.new_attention_workspace(rows + 1, hq, hkv, d, budget, cuda),
        )

    # Static inputs the host rewrites before every step.
    q = torch.empty((rows + 1, hq, d), dtype=dt, device=cuda)
    k = torch.empty((rows + 1, hkv, d), dtype=dt, device=cuda)
    v = torch.empty((rows + 1, hkv, d), dtype=dt, device=cuda)
    abs_pos = torch.empty(rows + 1, dtype=torch.int64, device=cuda)

    def launch(st):
        capture.capture_raw_kv_rows(k, v, st["raw_k"], st["raw_v"], slots, abs_pos, st["rope"], tokens=rows,
                                    working_lens=st["lens"])
        attention.draft_linear_attention(q, k, v, st["out"], st["work_k"], st["work_v"], st["lens"], slots, None,
                                         scale=d ** -0.5, workspace=st["ws"])

    graphed, eager, warm = fresh(), fresh(), fresh()
    launch(warm)  # first calls outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch(graphed)
    # Capture records work without running it: the graphed state is still the initial one.
    torch.cuda.synchronize()
    _same(graphed["lens"].cpu(), lens0, "lens after capture")

    host_k, host_v, host_lens = work_k.clone(), work_v.clone(), lens0.tolist()
    for step in range(3):
        q.copy_(randn(q.shape, dt, g))
        k.copy_(randn(k.shape, dt, g))
        v.copy_(randn(v.shape, dt, g))
        abs_pos.copy_(torch.tensor([200 + step, 10 + step, 500 + step, 0], dtype=torch.int64))
        torch.cuda.synchronize()
        graph.replay()
        launch(eager)
        torch.cuda.synchronize()
        for name in ("work_k", "work_v", "lens", "raw_k", "raw_v", "rope", "out"):
            _same(graphed[name], eager[name], f"step {step}: {name}")
        assert attention.attention_status(graphed["ws"]) == 0
        # The oracle's step on the host copies.
        s = slots.tolist()
        pos = [host_lens[x] for x in s]
        expected = torch.empty((rows, hq, d), dtype=dt)
        O.draft_linear_attention(q[:rows].cpu(), k[:rows].cpu(), v[:rows].cpu(), d ** -0.5, expected, host_k, host_v,
                                 host_lens, s, pos)
        terms = attention_terms(q[:rows].cpu(), host_k, host_v, s, pos, d ** -0.5)
        assert_attention_close(graphed["out"][:rows].cpu(), expected, terms)
        assert graphed["lens"].cpu().tolist() == host_lens
        assert graphed["rope"][:rows].cpu().tolist() == pos
        for r, x in enumerate(s):
            assert torch.equal(graphed["raw_k"][x, int(abs_pos[r])].cpu(), k[r].cpu())
            assert torch.equal(graphed["raw_v"][x, int(abs_pos[r])].cpu(), v[r].cpu())
    assert attention.attention_epoch(graphed["ws"]) == 3


@pytest.mark.parametrize("path", ["chain", "fused", "lse-free", "lse-free fused"])
def test_retrieval_step_replayed_from_a_graph(cuda, path):
    """One retrieval step captured once, replayed with new queries and committed counts
    (the chain and the single launch, each with and without a supplied LSE)."""
    from ds355 import step

    g = gen(43)
    lens = [int(x) for x in torch.randint(3000, 20000, (12,), generator=g)]
    counts = [int(x) for x in torch.randint(0, 6, (12,), generator=g)]
    slots = [int(x) for x in torch.randperm(12, generator=g)]
    case = build_case(43, real_rows=12, pad_rows=4, target_lens=lens, query_len=5, counts=counts, hq=32, hkv=4,
                      head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=20000, slots=slots,
                      num_slots=12)
    rows = case["rows"]
    max_chunks = (max(case["tlens"]) + 63) // 64
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=cuda)  # noqa: E731
    counts_t, committed_t = i32(case["counts"]), i32(case["committed"])
    rows_t = step.VerifierRows(counts_t, i32(case["starts"]), i32(case["qlens"]), i32(case["tlens"]),
                               case["real_rows"])
    query = case["query"].to(cuda)
    slots_t = i32(case["slots"])  # every tensor a descriptor names stays alive with it

    def fresh():
        st = dict(
            scores=torch.zeros((rows, max_chunks), dtype=torch.float32, device=cuda),
            partials=torch.zeros((rows, max_chunks, 4), dtype=torch.float32, device=cuda),
            sel_ids=torch.zeros((12, 32), dtype=torch.int32, device=cuda),
            sel_count=torch.full((12,), -1, dtype=torch.int32, device=cuda),
            plan=torch.zeros((rows, 5 + 32), dtype=torch.int64, device=cuda),
            working_lens=torch.zeros((12,), dtype=torch.int32, device=cuda),
            work_k=torch.full((12, 4, 2048, 128), float("nan"), dtype=torch.bfloat16, device=cuda),
        )
        st["work_v"] = torch.full_like(st["work_k"], float("nan"))
        lse_free = path.startswith("lse-free")
        if path.endswith("fused"):
            st["workspace"] = step.new_workspace(rows, max_chunks, 4, 2048, cuda)
        if lse_free:
            st["lse_partials"] = torch.zeros((rows, max_chunks, 32, 2), dtype=torch.float32, device=cuda)
            st["lse_out"] = torch.full((rows, 32), float("nan"), dtype=torch.float32, device=cuda)
        return st

    raw_k, raw_v = case["raw_k"].to(cuda), case["raw_v"].to(cuda)
    lse, key_cache, table = case["lse"].to(cuda), case["key_cache"].to(cuda), case["table"].to(cuda)
    cos_sin = case["cos_sin"].to(cuda)

    def desc_for(st):
        desc, _ = step.build_step_desc(
            snapshot=step.VerifierSnapshot(query, None if path.startswith("lse-free") else lse, key_cache, table,
                                           case["scale"]), rows=rows_t,
            scores=st["scores"], score_partials=st["partials"], sel_ids=st["sel_ids"], sel_count=st["sel_count"],
            slots=slots_t, committed_lens=committed_t, plan=st["plan"], working_lens=st["working_lens"],
            raw_key=raw_k, raw_value=raw_v, working_key=st["work_k"], working_value=st["work_v"],
            cos_sin_cache=cos_sin, rotary_dim=128, is_neox_style=True, chunk_size=64,
            history_budget=case["budget"], workspace=st.get("workspace"),
            lse_partials=st.get("lse_partials"), lse_out=st.get("lse_out"),
        )
        return desc

    graphed, eager, warm = fresh(), fresh(), fresh()
    graphed["desc"], eager["desc"], warm["desc"] = desc_for(graphed), desc_for(eager), desc_for(warm)
    step.launch(warm["desc"], cuda)  # first call outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step.launch(graphed["desc"], cuda)
    torch.cuda.synchronize()
    assert torch.isnan(graphed["work_k"]).all()  # capture records, it does not run

    outputs = ("scores", "sel_ids", "sel_count", "plan", "working_lens", "work_k", "work_v")
    if path.startswith("lse-free"):
        outputs += ("lse_out",)
    for replay in range(3):
        if replay:
            query.copy_(randn(tuple(query.shape), torch.bfloat16, g).to(cuda))
            new_counts = [int(x) for x in torch.randint(0, 6, (12,), generator=g)] + [0] * 4
            counts_t.copy_(i32(new_counts))
            committed_t.copy_(i32([tl - ql + min(max(c, 1), ql) for tl, ql, c in
                                   zip(case["tlens"], case["qlens"], new_counts)]))
        torch.cuda.synchronize()
        graph.replay()
        step.launch(eager["desc"], cuda)
        torch.cuda.synchronize()
        for name in outputs:
            _same(graphed[name], eager[name], f"replay {replay}: {name}")
        if path.endswith("fused"):
            assert step.workspace_status(graphed["workspace"]) == 0
            assert step.workspace_epoch(graphed["workspace"]) == replay + 1
        if replay == 0:  # the captured inputs: the oracle's step
            check_step(case, graphed)


def test_launches_use_torch_current_stream(cuda):
    """Every entry point launches on torch's current stream: the default one, a side stream, a capture."""
    from ds355 import _lib

    assert _lib.stream_handle(cuda) == torch.cuda.current_stream(cuda).cuda_stream
    side = torch.cuda.Stream(cuda)
    with torch.cuda.stream(side):
        assert _lib.stream_handle(cuda) == side.cuda_stream != torch.cuda.default_stream(cuda).cuda_stream
    x = torch.zeros(4, device=cuda)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert _lib.stream_handle(cuda) == torch.cuda.current_stream(cuda).cuda_stream
        x.add_(1)
    graph.replay()
    torch.cuda.synchronize()
    assert x.tolist() == [1.0] * 4
