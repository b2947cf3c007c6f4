"""GPU: seeded random batches through both implementations of the step.

Each seed draws one batch shape from the ranges the reference's own tests
span (tests/test_runtime.py, tests/test_retrieval_npu.py,
tests/test_linear_attention_batch_npu.py): rows 8-24 (the single launch's
range), ragged lengths from a few tokens to a few thousand, query lengths 1,
2 or 4 with committed counts 0..qlen (rows with 0 keep the previous
selection), graph padding rows, permuted slots among spare ones, chunk 16-64,
token budget 512-1024, GQA groups 1-8, head_dim 64 or 128, page sizes 16-128,
recent windows of one chunk or more, bf16 or fp16, neox or GPT-J rotation.
The chain is compared with the oracle (scores to the relative bar, the rest
bit-exact), the single launch with the chain bit for bit, and the compact
prefill alone (plan + gather in one launch, from the chain's selections) with
the chain's plans and working caches bit for bit.  With gather records, the
retrieval call moving each row's history prefix (the single launch) and the
compact prefill after it give the chain's plans and working caches bit for
bit, and a second compact prefill (everything held) changes nothing.
"""

import random

import pytest
import torch

from test_gpu_fused import _same
from test_gpu_step import build_case, check_step, run_gpu

pytestmark = pytest.mark.gpu


def _draw(seed):
    rnd = random.Random(1000 + seed)
    rows = rnd.randint(8, 24)
    pad = rnd.choice([0, 0, 3])
    chunk = rnd.choice([16, 32, 64])
    budget = rnd.choice([512, 1024])
    hkv, group = rnd.choice([(1, 8), (2, 4), (4, 8), (4, 2), (8, 1)])
    head_dim = rnd.choice([64, 128])
    block = rnd.choice([16, 64, 128])
    qlen = rnd.choice([1, 1, 2, 4])
    lens = [rnd.randint(qlen + 1, 6000) for _ in range(rows)]
    counts = [rnd.randint(0, qlen) if rnd.random() < 0.25 else rnd.randint(1, qlen) for _ in range(rows)]
    num_slots = rows + rnd.randint(0, 6)
    slots = rnd.sample(range(num_slots), rows)
    window = rnd.choice([None, chunk, 4 * chunk, 256])
    dtype = rnd.choice([torch.bfloat16, torch.float16])
    neox = rnd.random() < 0.7
    case = build_case(seed, real_rows=rows, pad_rows=pad, target_lens=lens, query_len=qlen, counts=counts,
                      hq=hkv * group, hkv=hkv, head_dim=head_dim, chunk=chunk, token_budget=budget,
                      block_size=block, lmax=max(lens) + 8, slots=slots, num_slots=num_slots, dtype=dtype,
                      neox=neox)
    label = (f"seed {seed}: rows {rows}+{pad}, qlen {qlen}, chunk {chunk}, budget {budget}, {group * hkv}/{hkv} "
             f"heads x {head_dim}, block {block}, window {window}, {dtype}, {'neox' if neox else 'gptj'}")
    return case, window, label


@pytest.mark.parametrize("seed", range(32))
def test_random_batches_chain_oracle_and_single_launch(cuda, seed):
    case, window, label = _draw(seed)
    print(label, flush=True)
    chain = run_gpu(case, cuda, path="chain", recent_window=window)
    check_step(case, chain, recent_window=window)
    fused = run_gpu(case, cuda, path="fused", recent_window=window)
    _same(chain, fused)
    # The compact prefill alone (plan + gather in one launch) from the chain's selections.
    from ds355 import step

    prefill = dict(chain)
    prefill.update(plan=torch.zeros_like(chain["plan"]), working_lens=torch.zeros_like(chain["working_lens"]),
                   work_k=torch.full_like(chain["work_k"], float("nan")),
                   work_v=torch.full_like(chain["work_v"], float("nan")),
                   sel_ids=chain["sel_ids"].clone(), sel_count=chain["sel_count"].clone())
    run_gpu(case, cuda, stages=step.PLAN, state=prefill, recent_window=window)
    _same_rebuild(chain, prefill)
    # Gather records: the prefix in the retrieval call, the rest in the compact prefill.
    records = (torch.zeros((case["num_slots"],), dtype=torch.int32, device=cuda),
               torch.zeros((case["num_slots"], case["token_budget"]), dtype=torch.int64, device=cuda))
    held = run_gpu(case, cuda, path="fused", stages=step.SCORE | step.SELECT | step.PREFIX, records=records,
                   derive_committed=True, recent_window=window)
    run_gpu(case, cuda, stages=step.PLAN, state=held, records=records, recent_window=window)
    _same_rebuild(chain, held)
    assert int((records[1] != 0).sum()) > 0 or max(case["committed"]) < 4 * case["chunk"]
    again = {k: v.clone() for k, v in held.items() if k in ("plan", "working_lens", "work_k", "work_v")}
    run_gpu(case, cuda, stages=step.PLAN, state=held, records=records, recent_window=window)
    _same_rebuild(again, held)


def _same_rebuild(want, got):
    for key in ("plan", "working_lens", "work_k", "work_v"):
        x, y = want[key], got[key]
        if x.dtype.is_floating_point:
            x, y = torch.nan_to_num(x), torch.nan_to_num(y)
        assert torch.equal(x, y), key
