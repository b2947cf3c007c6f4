"""GPU: the single-launch step gives the chain's results bit for bit.

Scores, selections, plans, working lengths and working caches of the fused
kernel are compared with the three-kernel chain on the same inputs (both
are checked against the oracle in test_gpu_step.py).  The workspace is
reused across launches and across batch shapes: its epoch advances by one
per launch and its status word stays 0.
"""

import pytest
import torch

from helpers import gen
from test_gpu_step import build_case, check_step, run_gpu

pytestmark = pytest.mark.gpu

KEYS = ("scores", "sel_ids", "sel_count", "plan", "working_lens", "work_k", "work_v")


def _same(a, b):
    for key in KEYS:
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
