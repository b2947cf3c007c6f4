"""GPU: the single-launch step gives the chain's results bit for bit.

Scores, selections, plans, working lengths and working caches of the fused
kernel are compared with the three-kernel chain on the same inputs (both
are checked against the oracle in test_gpu_step.py), with a supplied LSE
and without one (then the LSEs written to lse_out too).  The workspace is
reused across launches and across batch shapes: its epoch advances by one
per launch and its status word stays 0.
"""

import pytest
import torch

from helpers import gen
from test_gpu_step import build_case, check_step, run_gpu

pytestmark = pytest.mark.gpu

KEYS = ("scores", "sel_ids", "sel_count", "plan", "working_lens", "work_k", "work_v")
LSE_FREE_KEYS = KEYS + ("lse_out",)


def _same(a, b, keys=KEYS):
    for key in keys:
        x, y = a[key], b[key]
        if x.dtype.is_floating_point:
            assert torch.equal(x.isnan(), y.isnan()), key
            x, y = torch.nan_to_num(x), torch.nan_to_num(y)
        assert torch.equal(x, y), key


def _ragged(seed, rows, lo, hi, **kw):
    g = gen(seed)
    lens = [int(x) for x in torch.randint(lo, hi + 1, (rows,), generator=g)]
    args = dict(real_rows=rows, pad_rows=0, target_lens=lens, query_len=1, counts=[1] * rows, hq=32, hkv=4,
                head_dim=128, chunk=64, token_budget=2048, block_size=128, lmax=hi, slots=list(range(rows)),
                num_slots=rows)
    args.update(kw)
    return build_case(seed, **args)


def test_fused_equals_chain_bitwise(cuda):
    case = _ragged(11, 12, 100, 30000)
    chain = run_gpu(case, cuda, path="chain")
    fused = run_gpu(case, cuda, path="fused")
    _same(chain, fused)


def test_fused_rows_longer_than_one_poll_round(cuda):
    """Rows of 1031-1250 chunks: each selector reads its row's partials in rounds of 1024
    chunks while the scoring waves are still writing the later ones."""
    case = _ragged(31, 8, 33000, 40000, chunk=32, token_budget=1024)
    chain = run_gpu(case, cuda, path="chain")
    fused = run_gpu(case, cuda, path="fused")
    _same(chain, fused)


@pytest.mark.parametrize("seed,kw", [
    (32, dict(block_size=48)),
    (33, dict(hq=24, hkv=6, head_dim=64, block_size=80)),
])
def test_fused_pages_not_a_power_of_two(cuda, seed, kw):
    """Block sizes (48, 80) or KV head counts (6) that are not powers of two: the single
    launch's scoring resolves pages by division instead of shifts.  Oracle parity and the
    chain's bytes."""
    case = _ragged(seed, 10, 500, 9000, **kw)
    fused = run_gpu(case, cuda, path="fused")
    check_step(case, fused)
    chain = run_gpu(case, cuda, path="chain")
    _same(chain, fused)


def test_fused_repeated_launches_and_reused_workspace(cuda):
    """Three launches on one workspace, then another batch shape and layout in the same bytes."""
    from ds355 import step

    case = _ragged(12, 8, 2000, 12000)
    ref = run_gpu(case, cuda, path="chain")
    state = run_gpu(case, cuda, path="fused")
    for _ in range(2):
        state["work_k"].fill_(float("nan"))
        state["work_v"].fill_(float("nan"))
        state["sel_count"].fill_(-1)
        run_gpu(case, cuda, state=state, path="fused")
        _same(ref, state)
    assert step.workspace_epoch(state["workspace"]) == 3
    small = _ragged(13, 9, 500, 4000, hkv=2, hq=16, head_dim=64, chunk=32, token_budget=1024, block_size=64)
    small_ref = run_gpu(small, cuda, path="chain")
    small_state = run_gpu(small, cuda, path="chain")
    small_state["work_k"].fill_(float("nan"))
    small_state["work_v"].fill_(float("nan"))
    small_state["sel_count"].fill_(-1)
    small_state["workspace"] = state["workspace"]  # larger than needed: its epoch carries on
    run_gpu(small, cuda, state=small_state, path="fused")
    assert step.workspace_epoch(state["workspace"]) == 4
    _same(small_ref, small_state)


def test_unsupported_shape_with_workspace_runs_chain(cuda):
    """head_dim 96 is outside the fused kernel: the same call runs the chain and leaves the epoch."""
    case = _ragged(14, 4, 300, 5000, head_dim=96)
    chain = run_gpu(case, cuda, path="chain")
    state = run_gpu(case, cuda, path="fused", single_launch=False)
    _same(chain, state)


def test_pages_not_a_multiple_of_16_run_chain(cuda):
    """40-token blocks: a 16-token group can straddle two blocks, so scoring looks up
    each lane's page.  The single launch does not take such pages: the same call runs
    the chain, leaves the epoch, and matches the oracle."""
    case = _ragged(36, 9, 500, 6000, block_size=40)
    state = run_gpu(case, cuda, path="fused", single_launch=False)
    check_step(case, state)


def test_small_batch_with_workspace_runs_chain(cuda):
    """Below 8 rows the chain is faster; the same call runs it and leaves the epoch."""
    case = _ragged(15, 3, 2000, 9000)
    chain = run_gpu(case, cuda, path="chain")
    state = run_gpu(case, cuda, path="fused", single_launch=False)
    _same(chain, state)


@pytest.mark.parametrize("dtype,neox,head_dim", [(torch.float16, False, 128), (torch.float16, True, 64),
                                                 (torch.bfloat16, False, 64)])
def test_fused_fp16_and_gptj(cuda, dtype, neox, head_dim):
    """The single launch's other instances (fp16 caches, GPT-J rotary, head_dim 64): oracle parity and
    the chain's bytes."""
    case = _ragged(16, 9, 700, 9000, dtype=dtype, neox=neox, head_dim=head_dim, hq=16, hkv=2)
    fused = run_gpu(case, cuda, path="fused")
    check_step(case, fused)
    chain = run_gpu(case, cuda, path="chain")
    _same(chain, fused)


def test_selectors_gather_every_task(cuda):
    """The recovery path of the single launch, for every gather task: a scoring
    wave that stops waiting for its row's plan marks the task skipped and the
    last workgroup to finish does it.  Forced from the host (no scorer waits
    at all); the bytes equal the chain's and the status stays 0.  The next
    launch on the same workspace, without the flag, finds no stale skips."""
    from ds355 import step

    case = _ragged(17, 12, 1000, 20000)
    chain = run_gpu(case, cuda, path="chain")
    fused = run_gpu(case, cuda, path="fused", flags=step.SELECTORS_GATHER)
    _same(chain, fused)
    check_step(case, fused)
    for key in ("work_k", "work_v"):
        fused[key].fill_(float("nan"))
    fused["sel_count"].fill_(-1)
    run_gpu(case, cuda, state=fused, path="fused")
    _same(chain, fused)


def test_expired_wait_stays_with_its_launch(cuda):
    """A launch whose wait expired (forced from the host: every selector reports
    one) leaves its bit in the owner's status word and nothing in the launch
    word; the next launch on the same workspace runs its waits in full and
    equals the chain bit for bit, and clearing the owner's word works."""
    from ds355 import step

    case = _ragged(18, 10, 1000, 16000)
    chain = run_gpu(case, cuda, path="chain")
    state = run_gpu(case, cuda, path="fused", flags=step.EXPIRE_WAITS, expect_status=None)
    expired = step.workspace_status(state["workspace"])
    assert expired & 1  # bit 1 may join it: the launch's other waits stop early too
    for key in ("work_k", "work_v"):
        state[key].fill_(float("nan"))
    state["sel_count"].fill_(-1)
    run_gpu(case, cuda, state=state, path="fused", expect_status=expired)  # the owner has not cleared it
    _same(chain, state)
    step.clear_workspace_status(state["workspace"])
    for key in ("work_k", "work_v"):
        state[key].fill_(float("nan"))
    state["sel_count"].fill_(-1)
    run_gpu(case, cuda, state=state, path="fused")
    _same(chain, state)
    assert step.workspace_epoch(state["workspace"]) == 3


@pytest.mark.parametrize("seed,rows,lo,hi,kw", [
    (21, 12, 100, 30000, {}),
    (22, 9, 700, 9000, dict(hq=12, hkv=2, head_dim=64)),
    (23, 8, 20000, 40000, dict(chunk=32, token_budget=1024)),
    (24, 10, 500, 12000, dict(hq=64, hkv=8, head_dim=64, block_size=64)),
    (25, 9, 1000, 8000, dict(hq=16, hkv=1, head_dim=64, dtype=torch.float16)),
    (28, 9, 600, 9000, dict(hq=12, hkv=4, head_dim=64)),
    (29, 8, 800, 7000, dict(hq=28, hkv=4)),
    (30, 8, 500, 6000, dict(hq=16, hkv=2, head_dim=64, chunk=48, token_budget=1536, block_size=64)),
    (34, 9, 600, 9000, dict(block_size=48)),
    (35, 9, 600, 9000, dict(hq=24, hkv=6, head_dim=64, block_size=80, dtype=torch.float16)),
])
def test_lse_free_single_launch_equals_chain(cuda, seed, rows, lo, hi, kw):
    """Without a supplied LSE the single launch's selectors merge each row's mass
    words into its heads' LSEs with the chain's merge: scores, selections, plans,
    working caches and lse_out equal the chain's bit for bit, and match the
    oracle with the exact LSE.  Shapes: the headline's (ragged, 8 query heads per
    KV head); groups of 6 (three phases of two heads); 1250-chunk rows in
    32-token chunks (several load rounds per group and several chunk blocks);
    64 query heads (two rounds of words per chunk); one KV head of 16 in fp16;
    odd groups of 3 and 7 (one head per thread, 8-byte word reads); 48-token
    chunks at head_dim 64 (three 16-token groups per unit, two per batch); blocks
    of 48 and 80 tokens and 6 KV heads in fp16 (pages resolved by division)."""
    from oracle import diffspec_oracle as O

    case = _ragged(seed, rows, lo, hi, **kw)
    chain = run_gpu(case, cuda, path="chain", lse_free=True)
    fused = run_gpu(case, cuda, path="fused", lse_free=True)
    _same(chain, fused, LSE_FREE_KEYS)
    check_step(case, fused)
    rows_idx, q_index, _ = O.retrieval_rows(case["counts"], case["ends"], case["tlens"], case["real_rows"])
    torch.testing.assert_close(fused["lse_out"].cpu()[rows_idx], case["lse"][q_index], rtol=1e-5, atol=1e-4)


def test_lse_free_single_launch_takes_only_its_own_words(cuda):
    """The mass words carry their launch's tag.  One lse_partials buffer holds the
    chain's untagged words, then the words of a single launch on other queries;
    the next single launch (new queries again) waits for its own words: its
    results equal the chain's on its inputs, bit for bit."""
    from ds355 import step

    case = _ragged(26, 10, 2000, 16000)
    state = run_gpu(case, cuda, path="chain", lse_free=True)
    g = gen(27)
    for launch in range(3):
        query = torch.randn(tuple(case["query"].shape), generator=g).to(case["query"].dtype)
        other = dict(case, query=query)
        ref = run_gpu(other, cuda, path="chain", lse_free=True)
        state["query"] = query.to(cuda)
        for key in ("work_k", "work_v", "lse_out"):
            state[key].fill_(float("nan"))
        state["sel_count"].fill_(-1)
        state["scores"].zero_()
        run_gpu(other, cuda, state=state, path="fused", lse_free=True)
        _same(ref, state, LSE_FREE_KEYS)
    assert step.workspace_epoch(state["workspace"]) == 3


def test_lse_free_expired_wait_is_reported(cuda):
    """Without a supplied LSE a launch whose selectors report an expired wait
    (forced from the host) leaves the bit in the owner's word; the next launch
    equals the chain."""
    from ds355 import step

    case = _ragged(28, 9, 1000, 12000)
    chain = run_gpu(case, cuda, path="chain", lse_free=True)
    state = run_gpu(case, cuda, path="fused", lse_free=True, flags=step.EXPIRE_WAITS, expect_status=None)
    assert step.workspace_status(state["workspace"]) & 1
    step.clear_workspace_status(state["workspace"])
    for key in ("work_k", "work_v", "lse_out"):
        state[key].fill_(float("nan"))
    state["sel_count"].fill_(-1)
    run_gpu(case, cuda, state=state, path="fused", lse_free=True)
    _same(chain, state, LSE_FREE_KEYS)
