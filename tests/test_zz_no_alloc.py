"""GPU: ds_retrieval_step_static, the step whose scratch lives in the library's
static device array (for callers that cannot allocate), equals
ds_retrieval_step with caller buffers on the same inputs.

Each case makes two calls in a row through the C ABI, the second with a
smaller batch (fewer rows, shorter rows, so the static array's regions are
reused at another layout), on the single launch, the kernel chain and the
scoring without a supplied LSE.  Bar: bit-exact scores, selections, plans,
working lengths, working caches (NaN-filled outside the histories) and
LSEs: both entry points run the same kernels.  The status word stays 0.
"""

import pytest
import torch

from helpers import gen
from test_gpu_step import build_case, run_gpu

pytestmark = pytest.mark.gpu

KEYS = ("scores", "sel_ids", "sel_count", "plan", "working_lens", "work_k", "work_v")


def _case(seed, rows, lo, hi):
    g = gen(seed)
    lens = [int(x) for x in torch.randint(lo, hi + 1, (rows,), generator=g)]
    counts = [int(x) for x in torch.randint(1, 6, (rows,), generator=g)]
    slots = [int(x) for x in torch.randperm(rows, generator=g)]
    return build_case(seed, real_rows=rows, pad_rows=2, target_lens=lens, query_len=5, counts=counts, hq=32, hkv=4,
                      head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=hi, slots=slots,
                      num_slots=rows)


def _run_static(case, device, *, lse_free, check_free_memory):
    """The same buffers run_gpu makes, through ds_retrieval_step_static.

    With ``check_free_memory`` the device's free memory (hipMemGetInfo) must
    be the same before the call and after it has run: the entry point
    allocates nothing.  The first call of a process loads the code object
    that holds the static array, so only later calls are checked.
    """
    from ds355 import step

    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=device)  # noqa: E731
    rows = case["rows"]
    max_chunks = (max(case["tlens"]) + case["chunk"] - 1) // case["chunk"]
    st = dict(
        scores=torch.zeros((rows, max_chunks), dtype=torch.float32, device=device),
        sel_ids=torch.zeros((case["num_slots"], case["token_budget"] // case["chunk"]), dtype=torch.int32,
                            device=device),
        sel_count=torch.full((case["num_slots"],), -1, dtype=torch.int32, device=device),
        plan=torch.zeros((rows, 5 + case["token_budget"] // case["chunk"]), dtype=torch.int64, device=device),
        working_lens=torch.zeros((case["num_slots"],), dtype=torch.int32, device=device),
        work_k=torch.full((case["num_slots"], case["hkv"], case["token_budget"], case["head_dim"]), float("nan"),
                          dtype=case["dtype"], device=device),
        lse_out=torch.full((rows, case["hq"]), float("nan"), dtype=torch.float32, device=device),
    )
    st["work_v"] = torch.full_like(st["work_k"], float("nan"))
    # build_step_desc validates caller scratch; the static entry point does not use it.
    dummy_partials = torch.empty((rows, max_chunks, case["hkv"]), dtype=torch.float32, device=device)
    dummy_pairs = torch.empty((rows, max_chunks, case["hq"], 2), dtype=torch.float32, device=device)
    keep = dict(query=case["query"].to(device), lse=case["lse"].to(device), key_cache=case["key_cache"].to(device),
                table=case["table"].to(device), raw_k=case["raw_k"].to(device), raw_v=case["raw_v"].to(device),
                cos_sin=case["cos_sin"].to(device), counts=i32(case["counts"]), starts=i32(case["starts"]),
                qlens=i32(case["qlens"]), tlens=i32(case["tlens"]), slots=i32(case["slots"]),
                committed=i32(case["committed"]))
    desc, dev = step.build_step_desc(
        snapshot=step.VerifierSnapshot(keep["query"], None if lse_free else keep["lse"], keep["key_cache"],
                                       keep["table"], case["scale"]),
        rows=step.VerifierRows(keep["counts"], keep["starts"], keep["qlens"], keep["tlens"], case["real_rows"]),
        scores=st["scores"], score_partials=dummy_partials, sel_ids=st["sel_ids"], sel_count=st["sel_count"],
        slots=keep["slots"], committed_lens=keep["committed"], plan=st["plan"], working_lens=st["working_lens"],
        raw_key=keep["raw_k"], raw_value=keep["raw_v"], working_key=st["work_k"], working_value=st["work_v"],
        cos_sin_cache=keep["cos_sin"], rotary_dim=case["head_dim"], is_neox_style=case["neox"],
        chunk_size=case["chunk"], history_budget=case["budget"],
        lse_partials=dummy_pairs if lse_free else None, lse_out=st["lse_out"] if lse_free else None,
    )
    status = torch.zeros((1,), dtype=torch.int32, device=device)
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info(device)[0]
    step.launch_static(desc, dev, status)
    torch.cuda.synchronize()
    free_after = torch.cuda.mem_get_info(device)[0]
    if check_free_memory:
        assert free_after == free_before, f"free device memory moved by {free_before - free_after} bytes"
    assert int(status.item()) == 0
    return st


def _same(a, b, keys):
    for key in keys:
        x, y = a[key], b[key]
        if x.dtype.is_floating_point:
            assert torch.equal(x.isnan(), y.isnan()), key
            x, y = torch.nan_to_num(x), torch.nan_to_num(y)
        assert torch.equal(x, y), key


@pytest.mark.parametrize("kind,first,second", [
    ("single launch", (12, 1000, 20000), (9, 500, 6000)),
    ("chain", (4, 2000, 12000), (2, 300, 3000)),
    ("no LSE", (6, 1500, 15000), (3, 200, 4000)),
])
def test_static_scratch_step_equals_caller_buffers(cuda, kind, first, second):
    lse_free = kind == "no LSE"
    path = "fused" if kind == "single launch" else "chain"
    for call, (rows, lo, hi) in enumerate((first, second)):
        print(f"static scratch, {kind}, call {call + 1}: {rows} rows of {lo}..{hi} tokens", flush=True)
        case = _case(31 + 7 * call + len(kind), rows, lo, hi)
        expected = run_gpu(case, cuda, path=path, lse_free=lse_free,
                           single_launch=None if path == "fused" else False)
        got = _run_static(case, cuda, lse_free=lse_free, check_free_memory=call > 0)
        _same(expected, got, KEYS + (("lse_out",) if lse_free else ()))
