"""One retrieval step as a single launch chain (``ds_retrieval_step``).

score -> select (into per-slot state) -> plan -> gather/RoPE/write on the
current stream, with no host synchronisation.  This is the device-side
composition of diffspec/runtime.py:1211-1308 (row choice, committed query,
rejected-suffix cut, per-row selection), runtime.py:1737-1765 (plans) and
diffspec/compact_kv.py (gather).  Every argument is a device tensor or a host
integer known before the step; launch shapes depend only on the buffers'
sizes, so a step can be captured into a HIP graph.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


def _i32(name: str, t: torch.Tensor, n: int | None = None) -> torch.Tensor:
    if t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 tensor")
    if n is not None and t.numel() < n:
        raise ValueError(f"{name} has {t.numel()} entries, need {n}")
    return t


@dataclass
class VerifierSnapshot:
    """Target last-layer state used for scoring (runtime.py:841-878).

    query ``[tokens, Hq, D]``; lse viewed as ``[tokens, Hq]`` (any strides),
    or None: scoring then computes each query head's LSE over the row's
    scored tokens (the reference's ``chunk_attention_scores`` with
    ``softmax_lse=None``, runtime.py:321-322); key_cache ``[blocks,
    block_size, Hkv, D]``; block_table ``[rows, *]`` int32.
    """

    query: torch.Tensor
    lse: torch.Tensor | None
    key_cache: torch.Tensor
    block_table: torch.Tensor
    scale: float


@dataclass
class VerifierRows:
    """Per-row verifier metadata, int32 device tensors of ``batch_rows`` entries.

    ``counts`` = committed tokens (``valid_sampled_token_count``), ``query_start``
    / ``query_len`` = the row's query tokens, ``target_len`` = verifier KV
    length.  Rows at or beyond ``batch_size`` are graph padding.
    """

    counts: torch.Tensor
    query_start: torch.Tensor
    query_len: torch.Tensor
    target_len: torch.Tensor
    batch_size: int


SCORE, SELECT, PLAN, ALL = _lib.DS_STAGE_SCORE, _lib.DS_STAGE_SELECT, _lib.DS_STAGE_PLAN, _lib.DS_STAGE_ALL
PREFIX = _lib.DS_STAGE_PREFIX
SELECTORS_GATHER, EXPIRE_WAITS = _lib.DS_STEP_SELECTORS_GATHER, _lib.DS_STEP_EXPIRE_WAITS


def retrieval_step(*, reuse: dict | None = None, reuse_key=None, fixed_buffers: bool = False, **kwargs) -> None:
    """Run the stages of one step (see ``build_step_desc`` for the arguments).

    ``reuse`` (a dict the caller keeps) with ``reuse_key`` skips validation
    on repeated calls: the descriptor validated at the key's first call is
    kept and only its buffer addresses, scale and batch size are refreshed.
    The caller must change the key whenever anything but those changes
    (stages, shapes, strides, dtypes, devices, policy values, which optional
    buffers are given).  ``fixed_buffers`` says that, for one key, every
    buffer but the verifier snapshot's and the committed counts is the same
    tensor on every call (a runtime's own state): then only those addresses
    are refreshed.
    """
    if reuse is None or reuse_key is None:
        desc, device = build_step_desc(**kwargs)
    else:
        hit = reuse.get(reuse_key)
        if hit is None:
            if len(reuse) >= 64:
                reuse.clear()
            desc, device = build_step_desc(**kwargs)
            reuse[reuse_key] = (desc, device)
        else:
            desc, device = hit
            if fixed_buffers:
                snapshot, rows = kwargs.get("snapshot"), kwargs.get("rows")
                if snapshot is not None and desc.stages & (SCORE | SELECT):
                    desc.query, desc.lse = snapshot.query.data_ptr(), _lib.ptr(snapshot.lse)
                    desc.key_cache = snapshot.key_cache.data_ptr()
                    desc.block_table = snapshot.block_table.data_ptr()
                    desc.scale = float(snapshot.scale)
                    desc.counts = rows.counts.data_ptr()
            else:
                _set_pointers(desc, **{k: v for k, v in kwargs.items() if k in _POINTER_ARGS})
    launch(desc, device)


def launch(desc: _lib.StepDesc, device: torch.device, stages: int | None = None) -> None:
    """Launch a prebuilt descriptor on the current stream of ``device``.

    The descriptor holds raw device addresses: the tensors it was built from
    must stay alive and keep their storage.  ``stages`` overrides the
    descriptor's stage mask for this call.
    """
    if stages is not None:
        saved = desc.stages
        desc.stages = stages
    try:
        _lib.check(_lib.load().ds_retrieval_step(_lib.stream_handle(device), desc))
    finally:
        if stages is not None:
            desc.stages = saved


def launch_static(desc: _lib.StepDesc, device: torch.device, status: torch.Tensor | None = None) -> None:
    """Launch a prebuilt descriptor through ``ds_retrieval_step_static``.

    The step's scratch (score partials, the single launch's workspace, the
    mass words scored without an LSE) then lives in the library's static
    device array, so the
    descriptor's ``score_partials``, ``workspace`` and ``lse_partials`` are
    cleared for this call (the descriptor itself is not changed).  Nothing is
    allocated.  ``status`` (an int32 device word the caller clears) receives
    the status bits of a single launch whose bounded wait expired.  Calls
    that overlap on one GPU share that array and must be serialised.
    """
    local = _lib.StepDesc.from_buffer_copy(desc)
    local.score_partials = None
    local.workspace = None
    local.workspace_bytes = 0
    local.lse_partials = None
    if status is not None and (status.dtype != torch.int32 or status.device != device or status.numel() < 1):
        raise ValueError("status must be an int32 device word on the step's device")
    _lib.check(_lib.load().ds_retrieval_step_static(_lib.stream_handle(device), local, _lib.ptr(status)))


def build_step_desc(
    *,
    stages: int = ALL,
    snapshot: VerifierSnapshot | None,
    rows: VerifierRows | None,
    scores: torch.Tensor | None,
    score_partials: torch.Tensor | None = None,
    sel_ids: torch.Tensor,
    sel_count: torch.Tensor,
    slots: torch.Tensor,
    committed_lens: torch.Tensor | None,
    plan: torch.Tensor,
    working_lens: torch.Tensor | None,
    raw_key: torch.Tensor,
    raw_value: torch.Tensor,
    working_key: torch.Tensor,
    working_value: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    rotary_dim: int,
    is_neox_style: bool,
    chunk_size: int,
    history_budget: int,
    recent_window: int | None = None,
    row_active: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    lse_partials: torch.Tensor | None = None,
    lse_out: torch.Tensor | None = None,
    flags: int = 0,
    gather_records: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> tuple[_lib.StepDesc, torch.device]:
    """Validate and pack a step descriptor for ``stages`` (``SCORE | SELECT | PLAN``; ``ALL`` = one step).

    SCORE needs ``snapshot``; SCORE and SELECT need ``rows``, ``scores`` (a
    ``[batch_rows, max_chunks]`` fp32 buffer whose ``max_chunks`` covers
    ``ceil(max target_len / chunk_size)``; SELECT writes the final scores
    there) and ``score_partials`` (``[batch_rows, max_chunks, Hkv]`` fp32, the
    per-KV-head sums SCORE writes and SELECT reads).  PLAN writes ``plan`` and
    gathers.  ``workspace`` (from ``new_workspace``) lets a full step run as
    one launch when its shapes allow it; the results are the same.

    Without a snapshot LSE, SCORE needs ``lse_partials`` (``[batch_rows,
    max_chunks, Hq, 2]`` fp32 scratch: one 64-bit word per chunk and query
    head holding the chunk's mass) and ``lse_out`` (``[batch_rows, Hq]`` fp32,
    where each scored row's natural-log LSE is written).  With a workspace
    the full step still runs as the single launch; its words carry that
    workspace's launch tags, so keep one ``lse_partials`` per workspace.

    ``flags`` (tests only): ``SELECTORS_GATHER`` makes the single launch's
    scoring waves leave every gather task to the last workgroup to finish
    (the path of a task whose scoring wave stopped waiting for its plan; same
    results); ``EXPIRE_WAITS`` makes every selector report an expired wait
    (status bit 0, results not valid).

    ``gather_records`` = (``sel_gen`` ``[num_slots]`` int32, ``records``
    ``[num_slots, >= token_budget]`` int64, both zero-filled by the owner)
    lets a rebuild leave out the gather tasks whose working-cache bytes would
    not change (include/ds355.h: gather records): every stored selection
    increments the slot's generation, and the caller increments it when a
    different request takes the slot.  ``PREFIX`` in place of ``PLAN`` moves
    only the tasks wholly inside each row's history prefix (needs the
    records): the retrieval call can do that before the draft's prefill
    rewrites the rolling tail's raw rows.
    """
    if stages & ~(ALL | PREFIX):
        raise ValueError(f"unknown stage bits {stages:#x}")
    if stages & PREFIX and gather_records is None:
        raise ValueError("the PREFIX stage needs gather records")
    if stages & PREFIX and not stages & SELECT:
        raise ValueError("the PREFIX stage runs with SELECT (it needs the verifier rows)")
    uses_rows = bool(stages & (SCORE | SELECT))
    batch_rows = slots.numel()
    num_slots, max_model_len, heads, head_dim = raw_key.shape
    token_budget = working_key.shape[2]
    if raw_value.shape != raw_key.shape or working_value.shape != working_key.shape:
        raise ValueError("raw key/value must have matching 4-D shapes")
    if working_key.shape[0] != num_slots or working_key.shape[1] != heads or working_key.shape[3] != head_dim:
        raise ValueError("working cache slot, head and head dimensions must match raw KV")
    if not all(t.is_contiguous() for t in (raw_key, raw_value, working_key, working_value, plan)):
        raise ValueError("raw KV, working KV and plan must be contiguous")
    if plan.dtype != torch.int64 or plan.shape[0] != batch_rows:
        raise ValueError("plan must be int64 with one row per batch row")
    if cos_sin_cache.dtype != raw_key.dtype or cos_sin_cache.stride(1) != 1:
        raise ValueError("cos/sin cache must use the KV dtype with unit last stride")
    if cos_sin_cache.shape[0] < history_budget:
        raise ValueError("cos/sin cache must contain all local positions and rotary dimensions")
    _i32("slots", slots)
    if committed_lens is not None:
        _i32("committed_lens", committed_lens, batch_rows)
    elif stages & PLAN:
        raise ValueError("committed_lens is required (only a PREFIX rebuild with the verifier rows derives it)")
    _i32("sel_ids", sel_ids)
    _i32("sel_count", sel_count, num_slots)
    if sel_ids.shape[0] < num_slots:
        raise ValueError("sel_ids needs a row per slot")
    if working_lens is not None:
        _i32("working_lens", working_lens, num_slots)
    if row_active is not None:
        _i32("row_active", row_active, batch_rows)
    if workspace is not None and (workspace.dtype != torch.uint8 or not workspace.is_contiguous()
                                  or workspace.data_ptr() % 64 != 0):
        raise ValueError("workspace must be a contiguous, 64-byte aligned uint8 tensor (see new_workspace)")
    tensors = [sel_ids, sel_count, slots, committed_lens, plan, raw_key, raw_value, working_key, working_value,
               cos_sin_cache, working_lens, row_active, workspace]

    desc = _lib.StepDesc()
    desc.stages = stages
    desc.batch_size = batch_rows
    if uses_rows:
        if rows is None or scores is None:
            raise ValueError("scoring and selection need verifier rows and a score buffer")
        if scores.dtype != torch.float32 or scores.ndim != 2 or scores.shape[0] != batch_rows or not scores.is_contiguous():
            raise ValueError("scores must be a contiguous fp32 [batch_rows, max_chunks] buffer")
        for name in ("counts", "query_start", "query_len", "target_len"):
            _i32(name, getattr(rows, name), batch_rows)
        if not 0 <= rows.batch_size <= batch_rows:
            raise ValueError("batch_size must be between zero and batch_rows")
        if (score_partials is None or score_partials.dtype != torch.float32 or score_partials.ndim != 3
                or score_partials.shape[:2] != scores.shape or not score_partials.is_contiguous()):
            raise ValueError("score_partials must be a contiguous fp32 [batch_rows, max_chunks, kv_heads] buffer")
        tensors += [scores, score_partials, rows.counts, rows.query_start, rows.query_len, rows.target_len]
        desc.num_kv_heads = score_partials.shape[2]
        desc.max_chunks = scores.shape[1]
    if uses_rows:
        if snapshot is None:
            raise ValueError("scoring and selection need the verifier snapshot (heads, scale)")
        q, lse, kc, bt = snapshot.query, snapshot.lse, snapshot.key_cache, snapshot.block_table
        if q.ndim != 3 or kc.ndim != 4 or q.shape[2] != kc.shape[3]:
            raise ValueError("query and key head dimensions must match")
        if q.shape[1] % kc.shape[2] != 0:
            raise ValueError("query heads must be divisible by KV heads")
        if q.stride(2) != 1 or q.stride(1) != q.shape[2] or kc.stride(3) != 1:
            raise ValueError("query and key cache rows must be contiguous")
        if lse is not None and (lse.dtype != torch.float32 or lse.ndim != 2 or lse.shape != q.shape[:2]):
            raise ValueError("target softmax LSE does not match target query shape")
        if lse is None and stages & SCORE:
            hq = q.shape[1]
            if (lse_partials is None or lse_partials.dtype != torch.float32 or not lse_partials.is_contiguous()
                    or lse_partials.shape != (batch_rows, scores.shape[1], hq, 2)):
                raise ValueError("without a softmax LSE, lse_partials must be a contiguous fp32 "
                                 "[batch_rows, max_chunks, query_heads, 2] buffer")
            if lse_out is None or (lse_out.dtype != torch.float32 or lse_out.ndim != 2
                                   or lse_out.shape != (batch_rows, hq) or lse_out.stride(1) != 1):
                raise ValueError("without a softmax LSE, lse_out must be fp32 [batch_rows, query_heads] "
                                 "with unit head stride")
            tensors += [lse_partials, lse_out]
            desc.lse_out_stride = lse_out.stride(0)
        if bt.dtype != torch.int32 or bt.ndim != 2 or bt.stride(1) != 1 or bt.shape[0] < batch_rows:
            raise ValueError("block_table must be int32 [rows, blocks] with unit last stride")
        if q.dtype != kc.dtype:
            raise ValueError("query and key cache must share a dtype")
        if score_partials.shape[2] != kc.shape[2]:
            raise ValueError("score_partials must have one column per KV head")
        tensors += [q, lse, kc, bt]
        desc.dtype = _lib.dtype_code(q.dtype)
        desc.q_stride = q.stride(0)
        if lse is not None:
            desc.lse_token_stride, desc.lse_head_stride = lse.stride(0), lse.stride(1)
        desc.k_block_stride, desc.k_token_stride, desc.k_head_stride = kc.stride(0), kc.stride(1), kc.stride(2)
        desc.block_size = kc.shape[1]
        desc.bt_stride = bt.stride(0)
        desc.num_q_heads, desc.num_kv_heads, desc.head_dim = q.shape[1], kc.shape[2], q.shape[2]
    device = _lib.require_gpu(*tensors)
    desc.batch_rows = batch_rows
    desc.sel_stride = sel_ids.stride(0)
    desc.plan_width = plan.shape[1]
    desc.kv_dtype = _lib.dtype_code(raw_key.dtype)
    desc.num_slots, desc.max_model_len, desc.draft_heads, desc.draft_head_dim = num_slots, max_model_len, heads, head_dim
    desc.token_budget = token_budget
    desc.cs_stride, desc.cs_rows = cos_sin_cache.stride(0), cos_sin_cache.shape[0]
    desc.rotary_dim, desc.is_neox_style = rotary_dim, 1 if is_neox_style else 0
    desc.chunk_size, desc.history_budget = chunk_size, history_budget
    desc.recent_window = chunk_size if recent_window is None else recent_window
    desc.workspace_bytes = 0 if workspace is None else workspace.numel()
    _set_pointers(desc, snapshot=snapshot, rows=rows, scores=scores, score_partials=score_partials, sel_ids=sel_ids,
                  sel_count=sel_count, slots=slots, committed_lens=committed_lens, plan=plan,
                  working_lens=working_lens, raw_key=raw_key, raw_value=raw_value, working_key=working_key,
                  working_value=working_value, cos_sin_cache=cos_sin_cache, row_active=row_active,
                  workspace=workspace, lse_partials=lse_partials, lse_out=lse_out)
    if flags & ~(SELECTORS_GATHER | EXPIRE_WAITS):
        raise ValueError(f"unknown step flags {flags:#x}")
    if gather_records is not None:
        gen, records = gather_records
        _i32("sel_gen", gen, num_slots)
        if (records.dtype != torch.int64 or records.ndim != 2 or records.shape[0] < num_slots
                or records.shape[1] < token_budget or records.stride(1) != 1):
            raise ValueError("gather records must be int64 [num_slots, >= token_budget] with unit last stride")
        _lib.require_gpu(gen, records)
        desc.sel_gen, desc.gather_rec, desc.rec_stride = gen.data_ptr(), records.data_ptr(), records.stride(0)
    if _lib.DEBUG_CHECKS and stages & (PLAN | PREFIX):
        check_distinct_slots(slots, num_slots, row_active)
    desc.flags = flags
    return desc, device


def check_distinct_slots(slots: torch.Tensor, num_slots: int, row_active: torch.Tensor | None = None) -> None:
    """The plan stage's precondition (diffspec/compact_kv.py:199-205): no two
    re-gathered rows share a slot.  Rows whose slot is outside ``[0,
    num_slots)`` are graph padding.  Reads ``slots`` back (host
    synchronisation): run when ``DS355_DEBUG_CHECKS`` is set."""
    values = slots.detach().to("cpu").tolist()
    active = None if row_active is None else row_active.detach().to("cpu").tolist()
    seen: dict[int, int] = {}
    for r, slot in enumerate(values):
        if not 0 <= slot < num_slots or (active is not None and not active[r]):
            continue
        if slot in seen:
            raise ValueError(f"rows {seen[slot]} and {r} share slot {slot}; slots must be distinct")
        seen[slot] = r


_POINTER_ARGS = frozenset((
    "snapshot", "rows", "scores", "score_partials", "sel_ids", "sel_count", "slots", "committed_lens", "plan",
    "working_lens", "raw_key", "raw_value", "working_key", "working_value", "cos_sin_cache", "row_active",
    "workspace", "lse_partials", "lse_out"))


def _set_pointers(desc: _lib.StepDesc, *, snapshot=None, rows=None, scores=None, score_partials=None, sel_ids,
                  sel_count, slots, committed_lens, plan, working_lens=None, raw_key, raw_value, working_key,
                  working_value, cos_sin_cache, row_active=None, workspace=None, lse_partials=None,
                  lse_out=None) -> None:
    """The descriptor's buffer addresses, scale and batch size: everything a
    validated descriptor takes from the call rather than from the shapes."""
    p = _lib.ptr
    if desc.stages & (SCORE | SELECT):
        desc.scores, desc.score_partials = scores.data_ptr(), score_partials.data_ptr()
        desc.counts, desc.query_start = rows.counts.data_ptr(), rows.query_start.data_ptr()
        desc.query_len, desc.target_len = rows.query_len.data_ptr(), rows.target_len.data_ptr()
        desc.batch_size = rows.batch_size
        lse = snapshot.lse
        desc.query, desc.lse = snapshot.query.data_ptr(), p(lse)
        desc.key_cache, desc.block_table = snapshot.key_cache.data_ptr(), snapshot.block_table.data_ptr()
        desc.scale = float(snapshot.scale)
        if lse is None and desc.stages & SCORE:
            desc.lse_partials, desc.lse_out = lse_partials.data_ptr(), lse_out.data_ptr()
    else:
        desc.batch_size = desc.batch_rows
    desc.sel_ids, desc.sel_count, desc.slots = sel_ids.data_ptr(), sel_count.data_ptr(), slots.data_ptr()
    desc.committed_lens, desc.plan, desc.working_lens = p(committed_lens), plan.data_ptr(), p(working_lens)
    desc.raw_key, desc.raw_value = raw_key.data_ptr(), raw_value.data_ptr()
    desc.working_key, desc.working_value = working_key.data_ptr(), working_value.data_ptr()
    desc.cos_sin, desc.row_active, desc.workspace = cos_sin_cache.data_ptr(), p(row_active), p(workspace)


def workspace_bytes(batch_rows: int, max_chunks: int, num_kv_heads: int, token_budget: int) -> int:
    """Bytes of the single-launch step's workspace for these buffer sizes."""
    return int(_lib.load().ds_step_workspace_bytes(batch_rows, max_chunks, num_kv_heads, token_budget))


def new_workspace(batch_rows: int, max_chunks: int, num_kv_heads: int, token_budget: int,
                  device: torch.device) -> torch.Tensor:
    """A zero-filled workspace; keep it for the life of the buffers (one step at a time)."""
    n = workspace_bytes(batch_rows, max_chunks, num_kv_heads, token_budget)
    if n <= 0:
        raise ValueError("batch_rows, max_chunks, num_kv_heads and token_budget must be positive")
    return torch.zeros((n,), dtype=torch.uint8, device=device)


def workspace_epoch(workspace: torch.Tensor) -> int:
    """Number of single-launch steps completed on this workspace (synchronises)."""
    return int(workspace[:4].view(torch.int32).item()) & 0xFFFFFFFF


def workspace_launch_status(workspace: torch.Tensor) -> int:
    """Header word 3, the running launch's own status bits: 0 between launches (synchronises)."""
    return int(workspace[12:16].view(torch.int32).item()) & 0xFFFFFFFF


def workspace_status(workspace: torch.Tensor) -> int:
    """Status word: 0 unless a bounded wait of a single-launch step on this
    workspace expired since it was created or last cleared (synchronises).
    Bit 0: score partials, bit 1: gather tasks."""
    return int(workspace[8:12].view(torch.int32).item()) & 0xFFFFFFFF


def clear_workspace_status(workspace: torch.Tensor) -> None:
    """Zero the status word, stream-ordered (a fill kernel, no host synchronisation)."""
    workspace[8:12].zero_()
