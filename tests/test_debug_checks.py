"""Host checks of the plan preconditions the reference leaves to its callers
(diffspec/compact_kv.py:199-205: distinct slots, in-range entries), run when
DS355_DEBUG_CHECKS is set.  CPU only: they work on host copies."""

import pytest
import torch

from ds355 import compact_kv, step
from helpers import O


def _plan(rows, token_budget=16, chunk=2):
    return O.pad_plan(rows, token_budget, chunk)


def test_valid_plans_pass():
    plans = [O.history_plan(1, [0, 2, 5], 11, 2, 8), O.history_plan(0, None, 20, 2, 8), [3, 0, 0, 0, 0]]
    compact_kv.check_plan_preconditions(_plan(plans), num_slots=4, max_model_len=32, token_budget=16, chunk_size=2)
    step.check_distinct_slots(torch.tensor([2, 0, -1, 7, 1], dtype=torch.int32), num_slots=4)


def test_duplicate_slots_are_refused():
    plans = [O.history_plan(1, [0, 2, 5], 11, 2, 8), O.history_plan(1, None, 20, 2, 8)]
    with pytest.raises(ValueError, match="share slot 1"):
        compact_kv.check_plan_preconditions(_plan(plans), num_slots=4, max_model_len=32, token_budget=16,
                                            chunk_size=2)
    # A row that is not re-gathered may share its slot (it writes nothing).
    compact_kv.check_plan_preconditions(_plan(plans), num_slots=4, max_model_len=32, token_budget=16, chunk_size=2,
                                        row_active=torch.tensor([1, 0], dtype=torch.int32))
    with pytest.raises(ValueError, match="share slot 3"):
        step.check_distinct_slots(torch.tensor([3, 0, 3], dtype=torch.int32), num_slots=4)
    step.check_distinct_slots(torch.tensor([3, 0, 3], dtype=torch.int32), num_slots=4,
                              row_active=torch.tensor([1, 1, 0], dtype=torch.int32))


def test_out_of_range_entries_are_refused():
    good = O.history_plan(0, [0, 2, 5], 11, 2, 8)
    with pytest.raises(ValueError, match="slot 5 outside"):
        compact_kv.check_plan_preconditions(_plan([[5, *good[1:]]]), num_slots=4, max_model_len=32,
                                            token_budget=16, chunk_size=2)
    bad_chunk = list(good)
    bad_chunk[5] = 40  # chunk 40 starts at position 80 > max_model_len
    with pytest.raises(ValueError, match="prefix chunks outside"):
        compact_kv.check_plan_preconditions(_plan([bad_chunk]), num_slots=4, max_model_len=32, token_budget=16,
                                            chunk_size=2)
    with pytest.raises(ValueError, match="tail outside"):
        compact_kv.check_plan_preconditions(_plan([O.history_plan(0, None, 40, 2, 8)]), num_slots=4,
                                            max_model_len=32, token_budget=16, chunk_size=2)
