"""Host orchestration of DiffSpec retrieval and rebuild over the HIP chain.

``DiffSpecDraftCache`` mirrors the hot-path part of the reference's cache
(diffspec/runtime.py:596-1765): canonical slots, the verifier snapshot, the
retrieval cadence and skip rules, and the working-cache rebuild.  The
per-row Python loops, the ``counts.to("cpu")`` synchronisation and the
host-built plan of the reference are replaced by device state
(``sel_ids`` / ``sel_count`` / ``working_lens``) and the stage-split launch
chain of ``ds355.step``; host metadata that the reference already holds as
Python lists (query ends, verifier lengths, slots) is uploaded through a
small ring of pinned staging buffers with non-blocking copies.

Linear draft attention over the working cache (``forward_attention``) runs
as one launch of ``ds355.attention``; the raw pre-RoPE K/V capture of draft
tokens and the graph-safe RoPE input (``capture_raw_kv``,
``graph_safe_rope_positions``) as one launch of ``ds355.capture``.  The
adaptive retrieval cadence (``DiffSpecAdaptiveController``) is kept; tree
drafting is outside this module.
"""

from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib
from . import attention as _attention
from . import capture as _capture
from . import step as _step
from .plan import history_budget as _history_budget
from .plan import plan_width as _plan_width


@dataclass(frozen=True)
class DiffSpecSettings:
    """Field order and meaning of diffspec/runtime.py:18-41.

    ``recent_window`` is the only field the reference's settings lack; the
    cache reads it with ``getattr``, so the reference's own 7-field settings
    object works unchanged.
    """

    chunk_size: int
    token_budget: int
    retrieval_interval: int
    max_tree_nodes: int
    max_tree_depth: int
    tree_threshold: float
    adaptive_profile: bool
    recent_window: int | None = None  # None: one chunk, the reference's tail

    @classmethod
    def from_vllm_config(cls, vllm_config: Any) -> "DiffSpecSettings":
        """The speculative config's DiffSpec fields, mapped as diffspec/runtime.py:28-41 does.

        An optional ``diffspec_recent_window`` on the speculative config sets
        the rolling window; without it the window is one chunk.
        """
        spec = vllm_config.speculative_config
        if spec is None or not spec.use_diffspec():
            raise ValueError("DiffSpec settings require an enabled DiffSpec policy")
        return cls(
            chunk_size=spec.diffspec_chunk_size,
            token_budget=spec.diffspec_token_budget,
            retrieval_interval=spec.diffspec_retrieval_interval,
            max_tree_nodes=spec.diffspec_max_tree_nodes,
            max_tree_depth=spec.num_speculative_tokens,
            tree_threshold=spec.diffspec_tree_threshold,
            adaptive_profile=spec.diffspec_adaptive_profile,
            recent_window=getattr(spec, "diffspec_recent_window", None),
        )


@dataclass(frozen=True)
class DiffSpecTreeProfile:
    """A draft-tree size (diffspec/runtime.py:52-55)."""

    max_nodes: int
    max_depth: int


class DiffSpecAdaptiveController:
    """Retrieval cadence of diffspec/runtime.py:530-593.

    With ``adaptive`` set, every retrieval compares the first scored row's
    chunk selection with the one it replaced.  An overlap (intersection over
    union) of at least 0.9, with the accepted length not below 90% of the
    previous retrieval's, doubles the interval up to 32 cycles; anything else
    returns it to the configured base.  Tree profiles (``profile``,
    ``observe_cycle``) serve the reference's tree drafting, which this cache
    never proposes; they are kept so the proposer's reads see the same values.
    """

    PROFILES = (DiffSpecTreeProfile(16, 5), DiffSpecTreeProfile(32, 7), DiffSpecTreeProfile(50, 10))
    MAX_INTERVAL = 32

    def __init__(self, base_retrieval_interval: int, adaptive: bool) -> None:
        self.base_retrieval_interval = base_retrieval_interval
        self.retrieval_interval = base_retrieval_interval
        self.adaptive = adaptive
        self.profile = self.PROFILES[-1]
        self._throughput_ewma: dict[DiffSpecTreeProfile, float] = {}
        self._last_acceptance: float | None = None

    def observe_cycle(self, profile: DiffSpecTreeProfile, emitted_tokens: int, latency_seconds: float) -> None:
        """Throughput per tree profile; adaptive mode measures each, then keeps the best by 5%."""
        if latency_seconds <= 0:
            raise ValueError("latency_seconds must be positive")
        rate = emitted_tokens / latency_seconds
        self._throughput_ewma[profile] = 0.8 * self._throughput_ewma.get(profile, rate) + 0.2 * rate
        if not self.adaptive:
            return
        for candidate in self.PROFILES:
            if candidate not in self._throughput_ewma:
                self.profile = candidate
                return
        best = max(self._throughput_ewma, key=self._throughput_ewma.__getitem__)
        if self._throughput_ewma[best] > self._throughput_ewma.get(self.profile, 0.0) * 1.05:
            self.profile = best

    def observe_retrieval(self, previous_chunks: set[int], selected_chunks: set[int],
                          acceptance_length: float) -> None:
        union = previous_chunks | selected_chunks
        overlap = len(previous_chunks & selected_chunks) / len(union) if union else 1.0
        dropped = self._last_acceptance is not None and acceptance_length < 0.9 * self._last_acceptance
        if self.adaptive and overlap >= 0.9 and not dropped:
            self.retrieval_interval = min(2 * self.retrieval_interval, self.MAX_INTERVAL)
        else:
            self.retrieval_interval = self.base_retrieval_interval
        self._last_acceptance = acceptance_length


@dataclass
class DiffSpecRuntimeMetrics:
    """Retrieval counters of diffspec/runtime.py:65-116."""

    retrieval_count: int = 0
    retrieval_seconds: float = 0.0
    retrieval_attempts: int = 0
    retrieval_skipped_prefill: int = 0
    retrieval_skipped_no_snapshot: int = 0
    retrieval_skipped_interval: int = 0
    retrieval_skipped_no_committed_tokens: int = 0

    def observe_retrieval(self, elapsed_seconds: float) -> None:
        self.retrieval_count += 1
        self.retrieval_seconds += elapsed_seconds

    def snapshot(self) -> dict[str, float | int]:
        return {
            "retrieval_count": self.retrieval_count,
            "retrieval_attempts": self.retrieval_attempts,
            "retrieval_skipped_prefill": self.retrieval_skipped_prefill,
            "retrieval_skipped_no_snapshot": self.retrieval_skipped_no_snapshot,
            "retrieval_skipped_interval": self.retrieval_skipped_interval,
            "retrieval_skipped_no_committed_tokens": self.retrieval_skipped_no_committed_tokens,
            "retrieval_ms": self.retrieval_seconds / max(self.retrieval_count, 1) * 1.0e3,
        }


class _Staging:
    """Ring of pinned host buffers for small int32 row arrays (non-blocking H2D).

    On a GPU the copy and the ring's events go straight to the HIP runtime
    (a few microseconds less per upload than torch's copy and Event), or
    through torch's non-blocking copy and Event when the process's HIP
    runtime cannot be found by name.  The ring is cut into groups of
    ``group`` buffers with one event each, recorded after the group's last
    copy: the first buffer of a group is refilled only once the group's
    copies of the previous lap have run, so one upload in ``group`` records
    an event and the others record none.  Uploads go to one device buffer,
    so consumers are ordered by the stream.
    """

    def __init__(self, fields: int, rows: int, device: torch.device, depth: int = 32, group: int = 8) -> None:
        if depth % group:
            raise ValueError("the ring depth must be a multiple of the group size")
        pin = device.type == "cuda"
        self.pinned = pin
        self.host = [torch.zeros((fields, rows), dtype=torch.int32, pin_memory=pin) for _ in range(depth)]
        self.host_np = [h.numpy() for h in self.host]  # list -> pinned buffer without a temporary tensor
        self.group = group
        self.recorded = [False] * (depth // group)
        self.device = torch.zeros((fields, rows), dtype=torch.int32, device=device)
        self.index = 0
        self.hip = None
        self.events: list = []
        if pin:
            self.torch_device = device if device.index is not None else torch.device("cuda", torch.cuda.current_device())
            self.hip = _lib.hip_runtime()
            if self.hip is None:
                self.events = [torch.cuda.Event() for _ in range(depth // group)]
            else:
                for _ in range(depth // group):
                    ev = ctypes.c_void_p()
                    _lib.hip_check(self.hip.hipEventCreateWithFlags(ctypes.byref(ev), _lib.HIP_EVENT_DISABLE_TIMING),
                                   "hipEventCreateWithFlags")
                    self.events.append(ev)
            self.nbytes = fields * rows * 4
            self.host_ptr = [h.data_ptr() for h in self.host]
            self.device_ptr = self.device.data_ptr()

    def __del__(self) -> None:
        hip = getattr(self, "hip", None)
        if hip is not None:
            for ev in self.events:
                hip.hipEventDestroy(ev)

    def _wait(self, g: int) -> None:
        if self.hip is not None:
            _lib.hip_check(self.hip.hipEventSynchronize(self.events[g]), "hipEventSynchronize")
        else:
            self.events[g].synchronize()

    def drain(self) -> None:
        """Wait until every copy issued from the ring has run, so its host buffers may be released.

        Copies after a group's last recorded event are covered by a stream
        synchronisation; the ring is drained only when it is replaced.
        """
        if self.pinned:
            torch.cuda.current_stream(self.torch_device).synchronize()

    def upload(self, columns: list[list[int]]) -> torch.Tensor:
        i = self.index
        self.index = (i + 1) % len(self.host)
        g, k = divmod(i, self.group)
        if self.pinned and k == 0 and self.recorded[g]:
            self._wait(g)  # only waits if the GPU is a full ring behind
        buf = self.host_np[i]
        for f, values in enumerate(columns):
            if len(values):
                buf[f, : len(values)] = values
        if not self.pinned:
            self.device.copy_(self.host[i])
            return self.device
        hip = self.hip
        if hip is None:
            stream = torch.cuda.current_stream(self.torch_device)
            self.device.copy_(self.host[i], non_blocking=True)
            if k == self.group - 1:
                self.events[g].record(stream)
                self.recorded[g] = True
            return self.device
        stream = _lib.stream_handle(self.torch_device)
        _lib.hip_check(hip.hipMemcpyAsync(self.device_ptr, self.host_ptr[i], self.nbytes,
                                          _lib.HIP_MEMCPY_HOST_TO_DEVICE, stream), "hipMemcpyAsync")
        if k == self.group - 1:
            _lib.hip_check(hip.hipEventRecord(self.events[g], stream), "hipEventRecord")
            self.recorded[g] = True
        return self.device


WORKING_LENS = "working_lens"  # pending positions = the slots' device working lengths
# The retrieval call: score and select; with prefix_at_retrieval also every
# history row whose raw sources are final, all but the verifier's accepted
# positions.
RETRIEVAL_STAGES = _step.SCORE | _step.SELECT
PREFIX_RETRIEVAL_STAGES = _step.SCORE | _step.SELECT | _step.PREFIX
# Batches from which a step with a workspace runs as the single launch (the
# library's minimum, csrc/fused.hip kMinFusedRows), with or without an LSE.
SINGLE_LAUNCH_MIN_ROWS = 8


class DiffSpecDraftCache:
    """Canonical raw KV, bounded working cache and retrieval state.

    Constructor arguments follow diffspec/runtime.py:599-613.
    ``rotary_embedding`` supplies ``rotary_dim``, ``is_neox_style`` and
    either ``cos_sin_cache`` or ``_match_cos_sin_cache_dtype(x)``.
    ``lse_free_scoring`` (not in the reference) keeps a verifier snapshot
    whose attention backend returned no softmax LSE: scoring then computes
    each query head's LSE over the row's scored tokens in the same pass over
    K (the reference's ``chunk_attention_scores`` with ``softmax_lse=None``,
    runtime.py:321-322) and leaves it in ``scored_lse``.  Without it a
    snapshot with no LSE is dropped, as the reference does
    (runtime.py:850-851).
    """

    def __init__(
        self,
        settings: DiffSpecSettings,
        *,
        max_num_reqs: int,
        max_model_len: int,
        num_kv_heads: int,
        head_dim: int,
        target_num_layers: int,
        dtype: torch.dtype,
        device: torch.device,
        rotary_embedding: Any,
        target_cos_sin_cache: torch.Tensor | None = None,
        target_tensor_parallel_size: int = 1,
        max_batch_rows: int | None = None,
        lse_free_scoring: bool = False,
        prefix_at_retrieval: bool | None = None,
        recent_window: int | None = None,
    ) -> None:
        if target_tensor_parallel_size < 1:
            raise ValueError("Target tensor parallel size must be positive")
        self.settings = settings
        self.max_num_reqs = max_num_reqs
        self.max_model_len = max_model_len
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.target_last_layer = target_num_layers - 1
        self.target_tensor_parallel_size = target_tensor_parallel_size
        self.dtype = dtype
        self.device = torch.device(device)
        self.rotary_embedding = rotary_embedding
        self.target_cos_sin_cache = target_cos_sin_cache
        self.history_budget = _history_budget(settings.token_budget, settings.max_tree_depth, settings.chunk_size)
        # The rolling window: this argument, else the settings' field (the
        # reference's settings have none), else one chunk, the reference's tail.
        if recent_window is None:
            recent_window = getattr(settings, "recent_window", None)
        self.recent_window = settings.chunk_size if recent_window is None else int(recent_window)

        cache_shape = (max_num_reqs, max_model_len, num_kv_heads, head_dim)
        self.raw_key = torch.empty(cache_shape, dtype=dtype, device=self.device)
        self.raw_value = torch.empty_like(self.raw_key)
        working_shape = (max_num_reqs, num_kv_heads, settings.token_budget, head_dim)
        self.working_key = torch.empty(working_shape, dtype=dtype, device=self.device)
        self.working_value = torch.empty_like(self.working_key)

        # Per-slot selection state: sorted chunk ids and their count
        # (-1 = no selection yet, 0 = empty selection).
        capacity = settings.token_budget // settings.chunk_size
        self.sel_ids = torch.zeros((max_num_reqs, capacity), dtype=torch.int32, device=self.device)
        self.sel_count = torch.full((max_num_reqs,), -1, dtype=torch.int32, device=self.device)
        self.working_lens = torch.zeros((max_num_reqs,), dtype=torch.int32, device=self.device)
        # Gather records (include/ds355.h): each slot's selection generation,
        # and per gather task of its working cache what the cache holds, so
        # a compact prefill moves only what changed.  With
        # prefix_at_retrieval the retrieval call moves every task whose raw
        # rows are final before the draft's prefill (the history prefix and
        # the rolling tail up to the verifier's first query position), and the
        # compact prefill after it finds them recorded and moves the accepted
        # positions only.  That pays where the retrieval runs as the single
        # launch (16 rows x 40k tokens: 85.8 + 6.6 us against 62.6 + 31.6 us
        # for scoring and selection, then the whole rebuild); in the chain it
        # adds a launch (one 8k row: 21.1 + 6.4 against 15.7 + 8.3 us).  So by
        # default (None) it is on exactly when the retrieval is the single
        # launch: 8+ rows.  Between retrievals the compact prefill moves the
        # rolling tail.
        self.sel_gen = torch.zeros((max_num_reqs,), dtype=torch.int32, device=self.device)
        self.gather_records = torch.zeros((max_num_reqs, settings.token_budget), dtype=torch.int64,
                                          device=self.device)
        self._workspace: torch.Tensor | None = None  # single-launch retrieval, on first use
        self._workspace_heads = 0
        self.prefix_at_retrieval = prefix_at_retrieval

        self.max_batch_rows = max_batch_rows or max_num_reqs
        self.max_chunks = (max_model_len + settings.chunk_size - 1) // settings.chunk_size
        rows = self.max_batch_rows
        self.scores = torch.zeros((rows, self.max_chunks), dtype=torch.float32, device=self.device)
        self._score_partials: torch.Tensor | None = None  # [rows, max_chunks, target KV heads], on first use
        self.lse_free_scoring = lse_free_scoring
        # Without a snapshot LSE: the scoring pass's mass words (the library's
        # lse_partials, [rows, max_chunks, Hq, 2] fp32 = one 64-bit word per
        # chunk and head) and the computed natural-log LSE [rows, Hq], on
        # first use.
        self._lse_partials: torch.Tensor | None = None
        self.scored_lse: torch.Tensor | None = None
        self.plan = torch.zeros((rows, _plan_width(settings.token_budget, settings.chunk_size)),
                                dtype=torch.int64, device=self.device)
        self._rows_staging = _Staging(5, rows, self.device)
        self._plan_staging = _Staging(2, rows, self.device)
        self._attention_staging = _Staging(2, max_num_reqs, self.device)
        # Row order of slots as a device array, re-uploaded only when it changes
        # (a draft cycle's steps all use the same one).
        self._slot_map = _Staging(1, max_num_reqs, self.device)
        self._slot_map_list: list[int] | None = None

        self.controller = DiffSpecAdaptiveController(settings.retrieval_interval, settings.adaptive_profile)
        # Adaptive cadence compares a slot's selection before and after a
        # retrieval.  Both, and the committed counts, are copied to pinned
        # host memory on the stream; the comparison runs at the next
        # retrieval call, before the interval is read, which is the first
        # time the reference reads what it changes.  No synchronisation is
        # added to the retrieval itself.
        self._adaptive_pending: tuple | None = None
        self._adaptive_ids: torch.Tensor | None = None  # [before/after, slots, capacity]
        self._adaptive_sel_count: torch.Tensor | None = None  # [before/after, slots]
        self._adaptive_counts: torch.Tensor | None = None  # [rows]
        if settings.adaptive_profile:
            pin = self.device.type == "cuda"
            self._adaptive_ids = torch.zeros((2, max_num_reqs, capacity), dtype=torch.int32, pin_memory=pin)
            self._adaptive_sel_count = torch.zeros((2, max_num_reqs), dtype=torch.int32, pin_memory=pin)
            self._adaptive_counts = torch.zeros((self.max_batch_rows,), dtype=torch.int32, pin_memory=pin)
        self.metrics = DiffSpecRuntimeMetrics()
        self._request_slots: dict[str, int] = {}
        self._active_slots: list[int] = []
        self._retrieval_cycle = 0
        self._target_query: torch.Tensor | None = None
        self._target_lse: torch.Tensor | None = None
        self._target_key_cache: torch.Tensor | None = None
        self._target_block_tables: torch.Tensor | None = None
        self._target_query_ends: list[int] = []
        self._target_seq_lens: list[int] = []
        self._target_scale = 0.0
        self.target_is_prefill = True
        self.local_positions: torch.Tensor | None = None  # root positions of the last rebuild (device)
        # Pending linear draft attention (runtime.py:680-681): slots in row
        # order, and per-row local positions (a host list, a device tensor, or
        # WORKING_LENS = each slot's working length, read on the device).
        self._pending_request_indices: list[int] | None = None
        self._pending_local_positions: Any = None
        self._attention_workspace: torch.Tensor | None = None
        self._attention_workspace_for: tuple[int, int] | None = None  # (rows, heads) it was checked for
        # Draft cycle and capture state (runtime.py:677-699, 731-753, 1767-1794).
        self._cycle_open = False
        self._draft_step = 0
        self._compact_prefill = False
        self._rope_position_buffers: dict[torch.dtype, torch.Tensor] = {}
        self._rope_position_written: dict[torch.dtype, int] = {}
        self._capture_status = torch.zeros((1,), dtype=torch.int32, device=self.device)
        self._token_staging: _Staging | None = None  # token -> slot rows of populate_prefill
        self._step_descs: dict = {}  # validated step descriptors, reused while the shapes stay
        self._retrieval_rows: tuple | None = None  # verifier rows staged with the snapshot
        self._views: dict = {}  # slices of the cache's own buffers per batch size (slicing costs microseconds)
        self._attention_reuse: dict = {}
        self._capture_reuse: dict = {}
        # Verification is linear: this cache proposes no draft tree, so the
        # reference's tree activation (runtime.py:795-813) never fires and
        # these keep their "no tree" values (runtime.py:708-712).
        self.target_tree_active = False
        self.proposed_token_ids: torch.Tensor | None = None
        self.proposed_parent_indices: torch.Tensor | None = None
        self.proposed_depths: torch.Tensor | None = None
        self.proposed_depths_cpu: list[int] = []

    def retrieval_stages_for(self, batch_size: int) -> int:
        """The retrieval call's stages for a batch (see prefix_at_retrieval)."""
        prefix = self.prefix_at_retrieval
        if prefix is None:
            prefix = batch_size >= SINGLE_LAUNCH_MIN_ROWS
        return PREFIX_RETRIEVAL_STAGES if prefix else RETRIEVAL_STAGES

    @property
    def retrieval_interval(self) -> int:
        """Verifier cycles between retrievals (the controller's, diffspec/runtime.py:1206)."""
        return self.controller.retrieval_interval

    def _view(self, name: str, rows: int, make) -> torch.Tensor:
        """A slice of one of the cache's buffers, made once per batch size."""
        key = (name, rows)
        view = self._views.get(key)
        if view is None:
            view = self._views[key] = make()
        return view

    # -- draft cycle (runtime.py:731-753) -----------------------------------------------------------
    def begin_cycle(self, request_ids: list[str]) -> None:
        self.set_active_requests(request_ids)
        self._cycle_open = True
        self._draft_step = 0
        self._pending_request_indices = None
        self._pending_local_positions = None

    def end_cycle(self) -> None:
        self._cycle_open = False
        self._pending_request_indices = None
        self._pending_local_positions = None
        self._compact_prefill = False

    # -- slots (runtime.py:755-793) --------------------------------------------------------------
    def set_active_requests(self, request_ids: list[str]) -> None:
        """Keep canonical rows stable across batch reorder and cancellation."""
        active = set(request_ids)
        freed = []
        for request_id in list(self._request_slots):
            if request_id not in active:
                freed.append(self._request_slots.pop(request_id))
        if freed:
            index = torch.tensor(freed, dtype=torch.long).to(self.device)
            self.sel_count[index] = -1
            self.working_lens[index] = 0
            self.sel_gen[index] += 1  # the slot's records describe the request that left
        used = set(self._request_slots.values())
        free = iter(sorted(set(range(self.max_num_reqs)) - used))
        for request_id in request_ids:
            if request_id not in self._request_slots:
                try:
                    self._request_slots[request_id] = next(free)
                except StopIteration as error:
                    raise RuntimeError("DiffSpec canonical request slots are exhausted") from error
        self._active_slots = [self._request_slots[r] for r in request_ids]

    def begin_target_forward(self, request_ids: list[str]) -> None:
        """Discard a stale verifier snapshot before a new verifier pass."""
        self.set_active_requests(request_ids)
        self._target_query = None
        self._target_lse = None
        self._target_key_cache = None
        self._target_block_tables = None
        self._target_query_ends = []
        self._target_seq_lens = []
        self.target_is_prefill = True
        self._retrieval_rows = None

    def prepare_target_batch(self, request_ids: list[str], scheduled_spec_token_ids: dict[str, list[int]]) -> None:
        """Slots for the verifier batch; verification stays linear (runtime.py:795-813).

        The reference turns tree verification on only when a proposed tree
        was scheduled whole; this cache never proposes one.
        """
        del scheduled_spec_token_ids  # only consulted for a proposed tree
        self.set_active_requests(request_ids)
        self.target_tree_active = False

    def rewrite_target_positions(self, positions: Any, cumulative_query_lens: Any) -> None:
        """Tree-node positions (runtime.py:815-829): nothing to rewrite in linear verification."""
        del positions, cumulative_query_lens

    def accepted_target_token_indices(self) -> torch.Tensor:
        """Accepted tree-node offsets (runtime.py:831-834); no tree is ever verified here."""
        raise RuntimeError("DiffSpec tree has not been verified")

    def is_target_retrieval_layer(self, layer_index: int) -> bool:
        """The verifier layer whose query, LSE and K feed scoring: the last one (runtime.py:838-839)."""
        return layer_index == self.target_last_layer

    def clear_proposed_tree(self) -> None:
        """Drop a proposed tree (runtime.py:1526-1531); called before every linear proposal."""
        self.proposed_token_ids = None
        self.proposed_parent_indices = None
        self.proposed_depths = None
        self.proposed_depths_cpu = []

    # -- verifier snapshot (runtime.py:841-894) ---------------------------------------------------
    @staticmethod
    def _reshape_target_lse(query: torch.Tensor, softmax_lse: torch.Tensor) -> torch.Tensor:
        num_tokens, num_heads, _ = query.shape
        lse = softmax_lse.squeeze()
        if lse.ndim == 1 and num_tokens * num_heads == lse.numel():
            return lse.reshape(num_tokens, num_heads)
        if lse.shape == (num_tokens, num_heads):
            return lse
        if lse.shape == (num_heads, num_tokens):
            return lse.transpose(0, 1)  # a strided view: the kernel takes both strides
        if lse.numel() != num_tokens * num_heads:
            raise ValueError("target softmax LSE does not match target query shape")
        return lse.reshape(num_tokens, num_heads)

    def capture_target_attention(
        self,
        query: torch.Tensor,
        softmax_lse: torch.Tensor | None,
        key_cache: torch.Tensor | None,
        metadata: Any,
        scale: float,
    ) -> None:
        """Keep the last verifier layer's query, LSE and paged K (no copies of K).

        A missing LSE drops the snapshot unless ``lse_free_scoring`` is set.
        """
        if key_cache is None or (softmax_lse is None and not self.lse_free_scoring):
            return
        query_ends = list(getattr(metadata, "actual_seq_lengths_q", ()))
        seq_lens = list(getattr(metadata, "seq_lens_list", ()))
        block_tables = getattr(metadata, "block_tables", None)
        if not query_ends or not seq_lens or block_tables is None:
            return
        is_prefill = bool(getattr(metadata, "num_prefills", 1))
        lse = None if softmax_lse is None else self._reshape_target_lse(query, softmax_lse)
        if is_prefill:
            index = torch.tensor([end - 1 for end in query_ends], dtype=torch.long, device=query.device)
            lse = None if lse is None else lse.index_select(0, index)
            query = query.index_select(0, index)
            query_ends = list(range(1, len(query_ends) + 1))
        self._target_query = query.detach()
        self._target_lse = None if lse is None else lse.detach()
        self._target_key_cache = key_cache
        self._target_block_tables = block_tables[: len(seq_lens)]
        self._target_query_ends = query_ends
        self._target_seq_lens = seq_lens
        self._target_scale = scale
        self.target_is_prefill = is_prefill
        self._retrieval_rows = None if is_prefill else self._stage_retrieval_rows()

    def _stage_retrieval_rows(self) -> tuple | None:
        """Upload the verifier rows and compute the step key as soon as the snapshot exists.

        Both depend only on the snapshot and the active slots, so they run
        while the verifier's forward is still on the GPU, and the retrieval
        call only adds the committed counts and launches.  None where the
        retrieval call's own checks decide.
        """
        batch_size = len(self._active_slots)
        ends, seq_lens = self._target_query_ends, self._target_seq_lens
        if (batch_size == 0 or batch_size > self.max_batch_rows or len(ends) < batch_size
                or len(seq_lens) < batch_size or self._target_block_tables.shape[0] < batch_size
                or self.target_tensor_parallel_size > 1):
            return None
        ends = ends[:batch_size]
        starts = [0, *ends[:-1]]
        if max(seq_lens[:batch_size]) > self.max_chunks * self.settings.chunk_size:
            return None
        staged = self._rows_staging.upload([
            starts, [e - s for s, e in zip(starts, ends)], seq_lens[:batch_size], self._active_slots, [],
        ])
        key = self._step_key(self.retrieval_stages_for(batch_size), batch_size, batch_size,
                             self._cos_sin_cache(),
                             self._target_query, self._target_lse, self._target_key_cache, self._target_block_tables)
        return self._active_slots, staged, key

    # -- retrieval (runtime.py:1170-1334) ---------------------------------------------------------
    def accept_target_queries(self, valid_sampled_token_count: torch.Tensor, *, is_prefill: bool) -> None:
        """Retrieve context using the last committed verifier query per request."""
        self.metrics.retrieval_attempts += 1
        self._accept_target_queries(valid_sampled_token_count, is_prefill=is_prefill)

    def retrieval_status(self) -> dict[str, float | int]:
        """Counters plus slots holding a selection (reads the device state)."""
        return dict(
            self.metrics.snapshot(),
            retrieval_cycle=self._retrieval_cycle,
            selected_slots=int((self.sel_count >= 0).sum().item()),
            target_tensor_parallel_size=self.target_tensor_parallel_size,
        )

    def _observe_previous_retrieval(self) -> None:
        """Feed the last retrieval's first scored row to the cadence controller (runtime.py:1309-1331).

        That row is the first with a positive committed count; its selection
        before the retrieval (none or empty: no chunks) and after it are
        compared as chunk sets, with its accepted length ``count - 1``.  A
        retrieval with no committed row observes nothing, as the reference
        returns before scoring then.
        """
        pending, self._adaptive_pending = self._adaptive_pending, None
        if pending is None:
            return
        slots, batch_size, done = pending
        if done is not None:
            done.synchronize()  # recorded a verifier cycle ago: normally complete
        counts = self._adaptive_counts[:batch_size].tolist()
        first = next((i for i, c in enumerate(counts) if c > 0), None)
        if first is None:
            return
        slot = slots[first]
        chunks = [set(self._adaptive_ids[k, slot, : max(0, int(self._adaptive_sel_count[k, slot]))].tolist())
                  for k in (0, 1)]
        self.controller.observe_retrieval(chunks[0], chunks[1], float(max(0, counts[first] - 1)))

    def _copy_selection_state(self, which: int) -> None:
        """Every slot's selection (ids, then the count) into pinned host memory, on the stream."""
        self._adaptive_ids[which].copy_(self.sel_ids, non_blocking=True)
        self._adaptive_sel_count[which].copy_(self.sel_count, non_blocking=True)

    def _accept_target_queries(self, valid_sampled_token_count: torch.Tensor, *, is_prefill: bool) -> None:
        self._observe_previous_retrieval()
        if self._target_query is None or self._target_key_cache is None or self._target_block_tables is None:
            self.metrics.retrieval_skipped_no_snapshot += 1
            return
        if is_prefill:
            self.metrics.retrieval_skipped_prefill += 1
            return
        self._retrieval_cycle += 1
        if self._retrieval_cycle % self.retrieval_interval:
            self.metrics.retrieval_skipped_interval += 1
            return
        # Graph padding beyond the scheduler's requests is excluded (runtime.py:1211-1222).
        batch_size = len(self._active_slots)
        if (
            valid_sampled_token_count.numel() < batch_size
            or len(self._target_query_ends) < batch_size
            or len(self._target_seq_lens) < batch_size
            or self._target_block_tables.shape[0] < batch_size
        ):
            self.metrics.retrieval_skipped_no_snapshot += 1
            return
        if batch_size > self.max_batch_rows:
            raise RuntimeError("DiffSpec batch exceeds max_batch_rows")
        if self.target_tensor_parallel_size > 1:
            raise NotImplementedError("the chunk-score all-reduce across tensor-parallel ranks is not built")
        # A step where no row committed a token is skipped and counted, as
        # runtime.py:1253-1257 does, whenever that is known on the host: an
        # empty batch, or counts held in host memory.  Device counts stay on
        # the device (no synchronisation): such a step then runs, scores
        # nothing and leaves every selection as it was, with the same result
        # but without the counter.
        if batch_size == 0 or (valid_sampled_token_count.device.type == "cpu"
                               and int(valid_sampled_token_count.reshape(-1)[:batch_size].max()) <= 0):
            self.metrics.retrieval_skipped_no_committed_tokens += 1
            return
        # The rows and the key staged with this snapshot, unless the active
        # slots changed since.
        prepared, self._retrieval_rows = self._retrieval_rows, None
        if prepared is not None and prepared[0] is self._active_slots:
            staged, key = prepared[1], prepared[2]
        else:
            ends = self._target_query_ends[:batch_size]
            starts = [0, *ends[:-1]]
            lens = [e - s for s, e in zip(starts, ends)]
            if max(self._target_seq_lens[:batch_size]) > self.max_chunks * self.settings.chunk_size:
                raise ValueError("verifier length exceeds the score buffer (max_model_len)")
            staged = self._rows_staging.upload([
                starts, lens, self._target_seq_lens[:batch_size], self._active_slots, [],
            ])
            key = None
        # Whole staging rows serve any batch size (the kernels read the first
        # batch_size entries); int32 device counts are read where they are.
        counts = valid_sampled_token_count
        if (counts.dtype != torch.int32 or counts.device != self.device or not counts.is_contiguous()
                or counts.numel() < batch_size):
            counts = self._view("counts", batch_size, lambda: staged[4, :batch_size])
            counts.copy_(valid_sampled_token_count.reshape(-1)[:batch_size])  # device-side cast, no sync
        started = time.perf_counter()
        if self.controller.adaptive:
            self._copy_selection_state(0)
        q, lse, kc, bt = self._target_query, self._target_lse, self._target_key_cache, self._target_block_tables
        stages = self.retrieval_stages_for(batch_size)
        if key is None:
            key = self._step_key(stages, batch_size, batch_size, self._cos_sin_cache(), q, lse, kc, bt)
        hit = self._step_descs.get(key)
        if hit is not None:
            # The descriptor validated for this layout (what _launch refreshes).
            desc, device = hit
            desc.query, desc.lse, desc.key_cache, desc.block_table = (q.data_ptr(), _lib.ptr(lse), kc.data_ptr(),
                                                                      bt.data_ptr())
            desc.scale = float(self._target_scale)
            desc.counts = counts.data_ptr()
            _step.launch(desc, device)
        else:
            rows = _step.VerifierRows(
                counts=counts, query_start=self._view("qs", 0, lambda: staged[0]),
                query_len=self._view("ql", 0, lambda: staged[1]), target_len=self._view("tl", 0, lambda: staged[2]),
                batch_size=batch_size,
            )
            snapshot = _step.VerifierSnapshot(query=q, lse=lse, key_cache=kc, block_table=bt, scale=self._target_scale)
            self._launch(stages, batch_size, snapshot=snapshot, rows=rows,
                         slots=self._view("rs", batch_size, lambda: staged[3, :batch_size]), committed=None)
        if self.controller.adaptive:
            self._copy_selection_state(1)
            self._adaptive_counts[:batch_size].copy_(counts.reshape(-1)[:batch_size], non_blocking=True)
            done = None
            if self.device.type == "cuda":
                done = torch.cuda.Event()
                done.record(torch.cuda.current_stream(self.device))
            self._adaptive_pending = (list(self._active_slots), batch_size, done)
        self.metrics.observe_retrieval(time.perf_counter() - started)

    # -- rebuild (runtime.py:1349-1371, 1683-1765) ------------------------------------------------
    def prepare_compact_prefill(
        self, metadata: Any, num_tokens: int, *, committed_seq_lens: list[int] | torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Rebuild every active row's working cache at its committed root.

        ``committed_seq_lens`` (root position + 1 per row) may be a host list
        or an int32 device tensor.  Returns the rows' local root positions
        (the history lengths) as a device tensor; nothing is read back.
        """
        seq_lens = committed_seq_lens
        if seq_lens is None:
            seq_lens = list(getattr(metadata, "seq_lens_list", ()))
        if isinstance(seq_lens, list) and not seq_lens:
            raise RuntimeError("DiffSpec compact prefill requires sequence lengths")
        if not self._active_slots:
            raise RuntimeError("DiffSpec request slots have not been initialized")
        rows = num_tokens
        if rows > len(self._active_slots) or rows > self.max_batch_rows:
            raise RuntimeError("DiffSpec draft tensors omit active request rows")
        slots = self._active_slots[:rows]
        if isinstance(seq_lens, torch.Tensor):
            staged = self._plan_staging.upload([slots, []])
            staged[1, :rows].copy_(seq_lens.reshape(-1)[:rows])
        else:
            staged = self._plan_staging.upload([slots, list(seq_lens[:rows])])
        self._launch(_step.PLAN, rows, slots=self._view("ps", rows, lambda: staged[0, :rows]),
                     committed=self._view("pc", rows, lambda: staged[1, :rows]))
        self.local_positions = self._view("roots", rows, lambda: self.plan[:rows, 1])
        # The root token attends at its history length (runtime.py:1366-1369),
        # which the plan launch also stored as the slot's working length.
        self._pending_request_indices = list(slots)
        self._pending_local_positions = WORKING_LENS
        self._compact_prefill = True
        self._draft_step += 1
        return self.local_positions

    def populate_prefill(self, absolute_positions: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                         metadata: Any) -> None:
        """Write the draft's projected prefill rows into the raw cache (runtime.py:1336-1347).

        Token t goes to its request's slot (rows from ``metadata``'s query
        ends, runtime.py:1580-1594) at ``absolute_positions[t]``, every KV
        head, rejected tokens included (a later step overwrites them): one
        scatter launch, no RoPE input.  The next compact prefill's gather
        reads these rows, and runs after this launch on the same stream.
        """
        if not self._active_slots:
            raise RuntimeError("DiffSpec request slots have not been initialized")
        num_tokens = key.shape[0]
        if num_tokens == 0:
            return
        rows = self._request_indices(metadata, num_tokens)
        if max(rows) >= len(self._active_slots):
            raise RuntimeError("DiffSpec request slots have not been initialized")
        token_slots = [self._active_slots[r] for r in rows]
        staging = self._token_staging
        if staging is None or staging.device.shape[1] < num_tokens:
            capacity = max(num_tokens, 8 * self.max_batch_rows)
            if staging is not None:
                # Raw copies from the old ring's pinned buffers may still be
                # queued, and torch's host allocator does not know of them.
                staging.drain()
            staging = self._token_staging = _Staging(1, capacity, self.device)
        slots = staging.upload([token_slots])[0, :num_tokens]
        positions = absolute_positions.reshape(-1)[:num_tokens]
        if not positions.is_contiguous():
            positions = positions.contiguous()
        _capture.capture_raw_kv_rows(
            key, value, self.raw_key, self.raw_value, slots, positions, None, tokens=num_tokens,
            status=self._capture_status, reuse=self._capture_reuse)

    # -- raw KV capture and RoPE input (runtime.py:1580-1618, 1767-1877) -------------------------
    @staticmethod
    def _request_indices(metadata: Any, num_tokens: int) -> list[int]:
        """Token -> batch row from the query ends (runtime.py:1580-1594)."""
        query_ends = getattr(metadata, "actual_seq_lengths_q", None)
        starts = [0, *query_ends] if query_ends else metadata.query_start_loc.to("cpu").tolist()
        rows, row = [], 0
        for token in range(num_tokens):
            while row + 1 < len(starts) - 1 and token >= starts[row + 1]:
                row += 1
            rows.append(row)
        return rows

    def _device_slots(self, slots: list[int]) -> torch.Tensor:
        """``slots`` as an int32 device row (at most max_num_reqs entries).

        The copy is stream-ordered, so launches already queued keep reading
        the previous contents."""
        if self._slot_map_list != slots:
            self._slot_map.upload([slots])
            self._slot_map_list = list(slots)
        return self._view("slot_map", len(slots), lambda: self._slot_map.device[0, : len(slots)])

    def _rope_buffer(self, dtype: torch.dtype) -> torch.Tensor:
        buffer = self._rope_position_buffers.get(dtype)
        if buffer is None:
            buffer = torch.zeros((self.max_num_reqs * self.max_model_len,), dtype=dtype, device=self.device)
            self._rope_position_buffers[dtype] = buffer
        return buffer

    def capture_status(self) -> int:
        """Bit 0: a captured token's slot or absolute position was out of range (reads the device)."""
        return int(self._capture_status.item())

    def capture_raw_kv(
        self,
        layer_index: int,
        absolute_positions: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        metadata: Any = None,
    ) -> torch.Tensor | None:
        """Write the draft tokens' pre-RoPE K/V to the raw cache and, inside a
        draft cycle, arm the next attention and return the RoPE input.

        Linear drafting path of runtime.py:1797-1877: inside a cycle the rows
        are the active requests (graph padding beyond them is neither written
        nor given a position), their local positions are the slots' working
        lengths (the rebuilt history length for the root token) and the
        result is the cache-owned RoPE input that graph_safe_rope_positions
        would return, written by the same launch.  Outside a cycle every token
        goes to its request's slot (rows from ``metadata``'s query ends) and
        None is returned, as in the reference.  The "working cache exhausted"
        check the reference makes on host positions happens on the device
        (the attention's status word), since the positions never reach the
        host here.
        """
        if layer_index != 0:
            raise ValueError("DiffSpec draft cache only supports one layer")
        if not self._active_slots:
            raise RuntimeError("DiffSpec request slots have not been initialized")
        num_tokens = key.shape[0]
        prepared_root = self._compact_prefill
        if self._cycle_open:
            num_tokens = len(self._active_slots)
            if key.shape[0] < num_tokens or absolute_positions.numel() < num_tokens:
                raise RuntimeError("DiffSpec draft tensors omit active request rows")
            slots = self._active_slots[:num_tokens]
        else:
            if metadata is None:
                return None
            slots = [self._active_slots[r] for r in self._request_indices(metadata, num_tokens)]
        if prepared_root:
            self._compact_prefill = False
        if self._cycle_open and not prepared_root and self._draft_step == 0:
            # First draft step without a prepared root: rebuild first
            # (runtime.py:1857-1861); the plan leaves the root positions in
            # working_lens.
            seq_lens = list(getattr(metadata, "seq_lens_list", ())) if metadata is not None else []
            if not seq_lens:
                return None
            self.prepare_compact_prefill(metadata, num_tokens, committed_seq_lens=seq_lens)
            self._compact_prefill = False
            self._draft_step -= 1
        token_slots = self._device_slots(slots) if len(slots) <= self.max_num_reqs else torch.tensor(
            slots, dtype=torch.int32, device=self.device)
        dtype = absolute_positions.dtype
        buffer = self._rope_buffer(dtype)
        prev = self._rope_position_written.get(dtype, 0)
        if self._cycle_open:
            # The cache's own buffers (raw caches, RoPE buffer of this dtype,
            # working lengths, status, the slot row of this length) are fixed:
            # the launch layout is the draft tensors' layout and the counts.
            reuse_key = (key.shape, key.stride(), value.shape, value.stride(), key.dtype, value.dtype,
                         absolute_positions.shape, absolute_positions.stride(), dtype, num_tokens, prev)
            rope = _capture.capture_raw_kv_rows(
                key, value, self.raw_key, self.raw_value, token_slots, absolute_positions, buffer,
                tokens=num_tokens, working_lens=self.working_lens, prev_count=prev, status=self._capture_status,
                reuse=self._capture_reuse, reuse_key=reuse_key)
            self._rope_position_written[dtype] = absolute_positions.numel()
            self._pending_request_indices = list(slots)
            self._pending_local_positions = WORKING_LENS
            self._draft_step += 1
            return rope
        _capture.capture_raw_kv_rows(
            key, value, self.raw_key, self.raw_value, token_slots, absolute_positions[:num_tokens].contiguous(),
            buffer, tokens=num_tokens, prev_count=0, status=self._capture_status)
        # The launch wrote absolute positions into the RoPE buffer; its extent
        # is what graph_safe_rope_positions must clear next.
        self._rope_position_written[dtype] = max(prev, num_tokens)
        return None

    def graph_safe_rope_positions(
        self, absolute_positions: torch.Tensor, local_positions: torch.Tensor | None,
    ) -> torch.Tensor:
        """Cache-owned, stable RoPE input (runtime.py:1767-1794).

        The view capture_raw_kv returns is already this buffer and is returned
        as is; otherwise one launch copies the positions and zeroes the
        previous call's stale tail.
        """
        dtype = absolute_positions.dtype
        buffer = self._rope_buffer(dtype)
        count = absolute_positions.numel()
        if count > buffer.numel():
            raise RuntimeError("DiffSpec RoPE input exceeds its persistent buffer")
        if (local_positions is not None and local_positions.data_ptr() == buffer.data_ptr()
                and local_positions.numel() == count and self._rope_position_written.get(dtype, 0) == count):
            return local_positions.view(absolute_positions.shape)
        prev = self._rope_position_written.get(dtype, 0)
        local = None if local_positions is None else local_positions.to(dtype).contiguous()
        empty = self.raw_key.new_empty((0, self.num_kv_heads, self.head_dim))
        rope = _capture.capture_raw_kv_rows(
            empty, empty, self.raw_key, self.raw_value,
            torch.empty((0,), dtype=torch.int32, device=self.device), absolute_positions.contiguous(), buffer,
            tokens=0, local_positions=local, prev_count=prev)
        self._rope_position_written[dtype] = count
        return rope

    # -- linear draft attention (runtime.py:1853-1885, 2024-2134) ---------------------------------
    def prepare_draft_step(self, num_tokens: int | None = None) -> None:
        """Arm the next linear draft step: every active row attends at its
        slot's current working length (the non-root branch of runtime.py:1862-1871)."""
        if not self._active_slots:
            raise RuntimeError("DiffSpec request slots have not been initialized")
        rows = len(self._active_slots) if num_tokens is None else num_tokens
        if rows > len(self._active_slots):
            raise RuntimeError("DiffSpec draft tensors omit active request rows")
        self._pending_request_indices = self._active_slots[:rows]
        self._pending_local_positions = WORKING_LENS

    def has_pending_attention(self) -> bool:
        return self._pending_request_indices is not None and self._pending_local_positions is not None

    def forward_attention(
        self,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        scale: float,
        output: torch.Tensor,
    ) -> torch.Tensor:
        """Attend each pending row over its working cache; one launch, no host sync.

        Writes the new key/value at each row's local position, sets the
        slot's working length to position + 1 and zeroes output rows past the
        pending rows (graph padding), as runtime.py:2024-2134 does.
        """
        if not self.has_pending_attention():
            raise RuntimeError("DiffSpec attention called without prepared state")
        slots = self._pending_request_indices
        positions = self._pending_local_positions
        if isinstance(positions, str):
            positions = None
        rows = len(slots)
        heads = query.shape[1] if query.dim() == 3 else query.shape[1] // self.head_dim
        workspace = self._attention_workspace
        if self._attention_workspace_for != (rows, heads):
            need = _attention.attention_workspace_bytes(max(self.max_batch_rows, rows), heads, self.num_kv_heads,
                                                        self.head_dim, self.settings.token_budget)
            if workspace is None or workspace.numel() < need:
                workspace = _attention.new_attention_workspace(max(self.max_batch_rows, rows), heads,
                                                               self.num_kv_heads, self.head_dim,
                                                               self.settings.token_budget, self.device)
                self._attention_workspace = workspace
            self._attention_workspace_for = (rows, heads)
        if isinstance(positions, list):
            if len(positions) != rows:
                raise ValueError("one local position per pending row is required")
            if positions and max(positions) >= self.settings.token_budget:
                raise RuntimeError("DiffSpec working cache exhausted")
        slot_rows: Any = []
        if rows:
            slot_rows = self._device_slots(list(slots))
            if isinstance(positions, list):
                positions = self._attention_staging.upload([[], positions])[1, :rows]
        # Fixed here: the working caches and lengths, the workspace, the slot
        # row and the positions row of this length; the rest is the layout of
        # the caller's tensors.
        reuse_key = (query.shape, query.stride(), key.shape, key.stride(), value.shape, value.stride(),
                     output.shape, output.stride(), query.dtype, key.dtype, value.dtype, output.dtype, rows,
                     positions is None, float(scale), workspace.data_ptr())
        _attention.draft_linear_attention(
            query, key, value, output, self.working_key, self.working_value, self.working_lens,
            slot_rows, positions, scale=scale, workspace=workspace, reuse=self._attention_reuse,
            reuse_key=reuse_key if rows else None,
        )
        self._pending_request_indices = None
        self._pending_local_positions = None
        return output

    def _launch(
        self,
        stages: int,
        batch_rows: int,
        *,
        slots: torch.Tensor,
        committed: torch.Tensor | None,
        snapshot: _step.VerifierSnapshot | None = None,
        rows: _step.VerifierRows | None = None,
    ) -> None:
        rotary = self.rotary_embedding
        cos_sin = self._cos_sin_cache()
        partials = None
        if stages & (_step.SCORE | _step.SELECT):
            kv_heads = snapshot.key_cache.shape[2]
            if self._score_partials is None or self._score_partials.shape[2] != kv_heads:
                self._score_partials = torch.zeros((self.max_batch_rows, self.max_chunks, kv_heads),
                                                   dtype=torch.float32, device=self.device)
                self._views = {k: v for k, v in self._views.items() if k[0] != "partials"}
                self._step_descs.clear()  # they hold the old buffer's address
            partials = self._view("partials", batch_rows, lambda: self._score_partials[:batch_rows])
        lse_partials = lse_out = None
        if stages & _step.SCORE and snapshot.lse is None:
            q_heads = snapshot.query.shape[1]
            if self._lse_partials is None or self._lse_partials.shape[2] != q_heads:
                self._lse_partials = torch.zeros((self.max_batch_rows, self.max_chunks, q_heads, 2),
                                                 dtype=torch.float32, device=self.device)
                self.scored_lse = torch.zeros((self.max_batch_rows, q_heads), dtype=torch.float32,
                                              device=self.device)
                self._views = {k: v for k, v in self._views.items() if k[0] not in ("pairs", "lse_out")}
                self._step_descs.clear()
            lse_partials = self._view("pairs", batch_rows, lambda: self._lse_partials[:batch_rows])
            lse_out = self._view("lse_out", batch_rows, lambda: self.scored_lse[:batch_rows])
        workspace = None
        if stages & _step.SCORE and stages & _step.PREFIX:
            # Score, selection and the prefix gather as one launch where the
            # batch suits it (the library picks; the workspace allows it).
            kv_heads = snapshot.key_cache.shape[2]
            if self._workspace is None or self._workspace_heads != kv_heads:
                self._workspace = _step.new_workspace(self.max_batch_rows, self.max_chunks, kv_heads,
                                                      self.settings.token_budget, self.device)
                self._workspace_heads = kv_heads
                self._step_descs.clear()
            workspace = self._workspace
        key = self._step_key(stages, batch_rows, None if rows is None else rows.batch_size, cos_sin,
                             snapshot.query if snapshot is not None else None,
                             snapshot.lse if snapshot is not None else None,
                             snapshot.key_cache if snapshot is not None else None,
                             snapshot.block_table if snapshot is not None else None)
        hit = self._step_descs.get(key)
        if hit is not None:
            # The descriptor validated for this layout: only the verifier
            # snapshot's addresses, its scale and the committed counts change
            # (what retrieval_step(fixed_buffers=True) refreshes).
            desc, device = hit
            if snapshot is not None and stages & (_step.SCORE | _step.SELECT):
                desc.query, desc.lse = snapshot.query.data_ptr(), _lib.ptr(snapshot.lse)
                desc.key_cache, desc.block_table = snapshot.key_cache.data_ptr(), snapshot.block_table.data_ptr()
                desc.scale = float(snapshot.scale)
                desc.counts = rows.counts.data_ptr()
            _step.launch(desc, device)
            return
        _step.retrieval_step(
            reuse=self._step_descs, reuse_key=key, fixed_buffers=True,
            stages=stages, snapshot=snapshot, rows=rows,
            scores=self._view("scores", batch_rows, lambda: self.scores[:batch_rows])
            if stages & (_step.SCORE | _step.SELECT) else None,
            score_partials=partials,
            sel_ids=self.sel_ids, sel_count=self.sel_count, slots=slots, committed_lens=committed,
            plan=self._view("plan", batch_rows, lambda: self.plan[:batch_rows]), working_lens=self.working_lens,
            raw_key=self.raw_key, raw_value=self.raw_value,
            working_key=self.working_key, working_value=self.working_value,
            cos_sin_cache=cos_sin, rotary_dim=rotary.rotary_dim, is_neox_style=rotary.is_neox_style,
            chunk_size=self.settings.chunk_size, history_budget=self.history_budget,
            recent_window=self.recent_window, lse_partials=lse_partials, lse_out=lse_out, workspace=workspace,
            gather_records=(self.sel_gen, self.gather_records),
        )

    def _step_key(self, stages: int, batch_rows: int, batch_size: int | None, cos_sin: torch.Tensor,
                  q: torch.Tensor | None, lse: torch.Tensor | None, kc: torch.Tensor | None,
                  bt: torch.Tensor | None) -> tuple:
        """Everything but buffer addresses that a validated step descriptor
        depends on: the cache's own buffers keep their shapes, so the key is
        the stage mask, the batch and the verifier snapshot's layout."""
        rotary = self.rotary_embedding
        key = (stages, batch_rows, batch_size, cos_sin.shape, cos_sin.stride(0), rotary.rotary_dim,
               bool(rotary.is_neox_style))
        if q is not None:
            key += (q.shape, q.stride(), q.dtype, kc.shape, kc.stride(), kc.dtype, bt.shape, bt.stride(), bt.dtype,
                    None if lse is None else (lse.shape, lse.stride(), lse.dtype))
        return key

    def _cos_sin_cache(self) -> torch.Tensor:
        rotary = self.rotary_embedding
        match = getattr(rotary, "_match_cos_sin_cache_dtype", None)
        cache = match(self.raw_key) if match is not None else rotary.cos_sin_cache
        if cache.dtype != self.dtype or cache.device != self.device:
            cache = cache.to(device=self.device, dtype=self.dtype)
            rotary.cos_sin_cache = cache
        return cache
