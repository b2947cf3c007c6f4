"""Golden fixtures (tests/golden/): the reference's known answers and a small seeded step.

CPU: the oracle reproduces every known answer in kats.json (transcribed from
the reference plugin's tests, sources cited per entry) and regenerates
chain_small.npz bit for bit.  GPU: the HIP chain, on the fixture's inputs,
gives the fixture's outputs (scores within rtol 1e-3; selections, plans and
working caches bit-exact, untouched rows included), and the device
selection / plan / gather reproduce the known answers.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import O, assert_scores_close

GOLDEN = Path(__file__).resolve().parent / "golden"


def _kats(fn):
    return [k for k in json.loads((GOLDEN / "kats.json").read_text())["kats"] if k["fn"] == fn]


def _chain():
    z = np.load(GOLDEN / "chain_small.npz")
    cfg = json.loads(bytes(z["config"]).decode())
    bf = lambda name: torch.from_numpy(z[name].copy()).view(torch.bfloat16)  # noqa: E731
    t = lambda name: torch.from_numpy(z[name].copy())  # noqa: E731
    return z, cfg, bf, t


def test_golden_files_present_and_cited():
    data = json.loads((GOLDEN / "kats.json").read_text())["kats"]
    assert len(data) >= 16
    assert all(k["source"] for k in data)
    assert (GOLDEN / "chain_small.npz").exists() and (GOLDEN / "make_golden.py").exists()


@pytest.mark.parametrize("kat", _kats("history_budget"), ids=lambda k: str(k["inputs"]))
def test_oracle_history_budget_kats(kat):
    i = kat["inputs"]
    assert O.history_budget(i["token_budget"], i["max_tree_depth"], i["chunk_size"]) == kat["expected"]


@pytest.mark.parametrize("kat", _kats("select_context_chunks"), ids=lambda k: k["source"])
def test_oracle_selection_kats(kat):
    i = kat["inputs"]
    sel = O.select_context_chunks(torch.tensor(i["scores"]), i["seq_len"], i["chunk_size"], i["history_budget"])
    assert sel.chunk_indices.tolist() == kat["expected"]["chunk_indices"]
    assert sel.token_indices.tolist() == kat["expected"]["token_indices"]


@pytest.mark.parametrize("kat", _kats("history_indices"), ids=lambda k: str(k["inputs"]["history_end"]))
def test_oracle_history_kats(kat):
    i = kat["inputs"]
    got = O.history_indices(torch.tensor(i["selected"]), i["history_end"], i["chunk_size"], i["history_budget"])
    assert got.tolist() == kat["expected"]


@pytest.mark.parametrize("kat", _kats("history_indices+rebuild"), ids=lambda k: str(k["inputs"]["history_end"]))
def test_oracle_history_and_rebuild_value_kats(kat):
    i = kat["inputs"]
    idx = O.history_indices(torch.tensor(i["selected"]), i["history_end"], i["chunk_size"], i["history_budget"])
    assert idx.tolist() == kat["expected"]["indices"]
    raw_k = torch.zeros((1, 256, 1, 2))
    raw_v = torch.zeros((1, 256, 1, 2))
    raw_k[0, :, 0, 0] = torch.arange(256)
    raw_v[0, :, 0, 0] = torch.arange(256) + 1000
    work_k = torch.zeros((1, 1, 128, 2))
    work_v = torch.zeros((1, 1, 128, 2))
    lengths = O.rebuild_working_cache_per_request(
        raw_k, raw_v, work_k, work_v, [0], [i["history_end"] + 1], {0: torch.tensor(i["selected"])},
        torch.zeros((128, 2)), chunk_size=i["chunk_size"], budget=i["history_budget"], rotary_dim=0,
        is_neox_style=True)
    n = len(kat["expected"]["indices"])
    assert lengths == [n]
    assert work_k[0, 0, :n, 0].tolist() == kat["expected"]["working_key"]
    assert work_v[0, 0, :n, 0].tolist() == kat["expected"]["working_value"]


def test_oracle_regenerates_chain_fixture():
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    z, _, _, _ = _chain()
    arrays = mod._draw_chain(int(z["seed"][0]))["arrays"]
    for name, value in arrays.items():
        if value.dtype.kind == "f" and name in ("lse", "scores"):
            # Floating-point reductions (logsumexp, softmax sums) may round
            # differently on another host's vector units: within 4 ulps of fp32.
            np.testing.assert_allclose(value, z[name], rtol=5e-7, atol=0, err_msg=name)
        else:
            assert np.array_equal(value, z[name]), name


# -- GPU ------------------------------------------------------------------------------------------
@pytest.mark.gpu
def test_gpu_chain_matches_golden(cuda):
    from ds355 import step

    z, cfg, bf, t = _chain()
    rows, chunk, hkv, d, tb = cfg["rows"], cfg["chunk"], cfg["hkv"], cfg["d"], cfg["token_budget"]
    lengths = t("lengths").tolist()
    hb = int(z["history_budget"][0])
    dev = lambda x: x.to(cuda)  # noqa: E731
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=cuda)  # noqa: E731
    max_chunks = z["scores"].shape[1]
    scores = torch.zeros((rows, max_chunks), device=cuda)
    partials = torch.zeros((rows, max_chunks, hkv), device=cuda)
    sel_ids = torch.zeros((rows, tb // chunk), dtype=torch.int32, device=cuda)
    sel_count = torch.full((rows,), -1, dtype=torch.int32, device=cuda)
    plan = torch.zeros((rows, 5 + tb // chunk), dtype=torch.int64, device=cuda)
    nan_bits = torch.full((rows, hkv, tb, d), 0x7fc0, dtype=torch.int16)
    work_k = nan_bits.clone().view(torch.bfloat16).to(cuda)
    work_v = nan_bits.clone().view(torch.bfloat16).to(cuda)
    step.retrieval_step(
        snapshot=step.VerifierSnapshot(dev(bf("query")), dev(t("lse")), dev(bf("key_cache")), dev(t("block_table")),
                                       float(z["scale"][0])),
        rows=step.VerifierRows(i32([1] * rows), i32(list(range(rows))), i32([1] * rows), i32(lengths), rows),
        scores=scores, score_partials=partials, sel_ids=sel_ids, sel_count=sel_count, slots=dev(t("slots")),
        committed_lens=i32(lengths), plan=plan, working_lens=None, raw_key=dev(bf("raw_key")),
        raw_value=dev(bf("raw_value")), working_key=work_k, working_value=work_v, cos_sin_cache=dev(bf("cos_sin")),
        rotary_dim=d, is_neox_style=True, chunk_size=chunk, history_budget=hb, recent_window=cfg["recent_window"],
    )
    torch.cuda.synchronize()
    assert_scores_close(scores.cpu(), t("scores"))
    assert torch.equal(sel_count.cpu(), t("sel_count"))
    for s in range(rows):
        n = int(z["sel_count"][s])
        assert sel_ids[s, :n].cpu().tolist() == z["sel_ids"][s, :n].tolist()
    assert torch.equal(plan.cpu(), t("plan"))
    assert torch.equal(work_k.cpu().view(torch.int16), t("working_key"))
    assert torch.equal(work_v.cpu().view(torch.int16), t("working_value"))


@pytest.mark.gpu
@pytest.mark.parametrize("kat", _kats("select_context_chunks"), ids=lambda k: k["source"])
def test_gpu_selection_kats(cuda, kat):
    from ds355.selection import select_context_chunks

    i = kat["inputs"]
    sel = select_context_chunks(torch.tensor(i["scores"], device=cuda), i["seq_len"], i["chunk_size"],
                                i["history_budget"])
    assert sel.chunk_indices.cpu().tolist() == kat["expected"]["chunk_indices"]
    assert sel.token_indices.cpu().tolist() == kat["expected"]["token_indices"]


@pytest.mark.gpu
@pytest.mark.parametrize("kat", _kats("history_indices+rebuild"), ids=lambda k: str(k["inputs"]["history_end"]))
def test_gpu_plan_and_gather_value_kats(cuda, kat):
    """Device plan + gather with the identity rotation (rotary_dim 0) reproduce the rebuilt values."""
    from ds355.compact_kv import rebuild_compact_kv_from_plan
    from ds355.plan import build_history_plans

    i = kat["inputs"]
    chunk, hb, tb = i["chunk_size"], i["history_budget"], 128
    chunks = sorted({t // chunk for t in i["selected"]})
    sel_ids = torch.zeros((1, tb // chunk), dtype=torch.int32)
    sel_ids[0, :len(chunks)] = torch.tensor(chunks, dtype=torch.int32)
    plan = build_history_plans(
        sel_ids.to(cuda), torch.tensor([len(chunks)], dtype=torch.int32, device=cuda),
        torch.tensor([0], dtype=torch.int32, device=cuda),
        torch.tensor([i["history_end"] + 1], dtype=torch.int32, device=cuda),
        chunk_size=chunk, history_budget=hb, token_budget=tb)
    raw_k = torch.zeros((1, 256, 1, 2))
    raw_v = torch.zeros((1, 256, 1, 2))
    raw_k[0, :, 0, 0] = torch.arange(256)
    raw_v[0, :, 0, 0] = torch.arange(256) + 1000
    work_k = torch.zeros((1, 1, tb, 2), device=cuda)
    work_v = torch.zeros((1, 1, tb, 2), device=cuda)
    rebuild_compact_kv_from_plan(raw_k.to(cuda), raw_v.to(cuda), work_k, work_v, plan, torch.zeros((tb, 2), device=cuda),
                                 chunk_size=chunk, max_width=hb, rotary_dim=0, is_neox_style=True)
    torch.cuda.synchronize()
    n = len(kat["expected"]["indices"])
    assert int(plan[0, 1]) == n
    assert work_k[0, 0, :n, 0].cpu().tolist() == kat["expected"]["working_key"]
    assert work_v[0, 0, :n, 0].cpu().tolist() == kat["expected"]["working_value"]
