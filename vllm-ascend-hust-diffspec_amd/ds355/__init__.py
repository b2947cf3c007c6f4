"""ds355: MI355X (gfx950) DiffSpec draft-context retrieval.

Drop-in replacements for the reference plugin's hot path:

- ``ds355.kernels.paged_chunk_attention_scores``  (diffspec/kernels.py:95-150)
- ``ds355.selection.select_context_chunks``        (diffspec/runtime.py:348-414)
- ``ds355.plan.build_history_plans``               (diffspec/runtime.py:1713-1757)
- ``ds355.compact_kv.rebuild_compact_kv_from_plan`` (diffspec/compact_kv.py:184-242)
- ``ds355.step.retrieval_step``                    (one launch chain for a whole step)
- ``ds355.runtime.DiffSpecDraftCache``             (host orchestration, runtime.py:596-1765)

All device work runs in the HIP library ``libds355.so`` (C ABI in
``include/ds355.h``); there is no CPU fallback.
"""

__version__ = "0.1.0"
