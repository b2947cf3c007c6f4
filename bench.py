"""Benchmark: microseconds per DiffSpec retrieval step on one MI355X.

A step is one launch chain over a ragged batch: chunk scores (paged target
K, committed query, supplied LSE) -> per-request top-k selection -> history
plans -> gather of the selected pre-RoPE KV + RoPE at local positions +
working-cache write.  Inputs are synthetic (seeded N(0,1) bf16), resident in
HBM before timing, and rotated over several copies so consecutive steps do
not hit in the 256 MB Infinity Cache.

Prints ONE JSON line.  The default workload is the 16-request ragged batch
(context lengths uniform in [4096, 40960], 4 KV heads x 128, 32 query heads,
chunk 64, token budget 2048, K = 4 draft tokens -> 1984 history tokens).

Besides the step (value, roofline, per-stage kernel times, cpu_baseline) the
line carries the path's neighbours on the same inputs: the scores without a
supplied LSE (lse_free_scoring), the draft decode attention over the working
caches the step gathered (draft_attention), the raw-KV capture of one draft
token per row (draft_capture) and the host time of the runtime's calls over
whole draft cycles (runtime_host).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
import types
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "vllm-ascend-hust-diffspec_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
METRIC = "µs per retrieval step (16 req, 40k ctx) and achieved HBM GB/s vs peak, 1 GPU"

WORKLOADS = {
    # name: (rows, lengths spec, Hq, Hkv, D, chunk, token_budget, padding rows, qlen, permuted slots, reuse half)
    "single-8k": dict(rows=1, lens=("fixed", 8192), hq=32, hkv=4, d=128, chunk=64, budget=2048),
    "ragged16-40k": dict(rows=16, lens=("uniform", 4096, 40960), hq=32, hkv=4, d=128, chunk=64, budget=2048),
    "fixed16-40k": dict(rows=16, lens=("fixed", 40960), hq=32, hkv=4, d=128, chunk=64, budget=2048),
    "long4-128k": dict(rows=4, lens=("fixed", 131072), hq=32, hkv=4, d=128, chunk=32, budget=2048),
    "specmask16-pad32": dict(rows=16, lens=("uniform", 8192, 40960), hq=32, hkv=4, d=128, chunk=64, budget=2048,
                             pad=16, qlen=5, permute=True),
    "stress64": dict(rows=64, lens=("uniform", 2048, 40960), hq=64, hkv=8, d=128, chunk=128, budget=4096,
                     reuse_half=True, window=512),
}
RECENT_WINDOW = 256  # rolling recent-window tokens (stress64: 512)
DEFAULT_WORKLOAD = "ragged16-40k"
DRAFT_TOKENS = 4
BLOCK_SIZE = 128
ROPE_THETA = 1.0e6


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def build_inputs(spec, seed, device):
    """Seeded synthetic verifier batch + draft caches on `device`."""
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    rows = spec["rows"]
    pad = spec.get("pad", 0)
    qlen = spec.get("qlen", 1)
    kind = spec["lens"][0]
    if kind == "fixed":
        tlens = [spec["lens"][1]] * rows
    else:
        lo, hi = spec["lens"][1], spec["lens"][2]
        tlens = [int(x) for x in torch.randint(lo, hi + 1, (rows,), generator=g)]
    if qlen > 1:
        accepted = [int(x) for x in torch.randint(0, DRAFT_TOKENS + 1, (rows,), generator=g)]
        counts = [a + 1 for a in accepted]
    else:
        counts = [1] * rows
    slots = [int(x) for x in torch.randperm(rows, generator=g)] if spec.get("permute") else list(range(rows))
    hq, hkv, d, chunk = spec["hq"], spec["hkv"], spec["d"], spec["chunk"]
    total_rows = rows + pad
    qlens = [qlen] * rows + [1] * pad
    all_tlens = tlens + [1] * pad
    ends = [sum(qlens[: i + 1]) for i in range(total_rows)]
    starts = [0, *ends[:-1]]
    committed = [tl - ql + min(max(c, 1), ql) for tl, ql, c in zip(all_tlens, qlens, counts + [0] * pad)]
    pages = [(n + BLOCK_SIZE - 1) // BLOCK_SIZE for n in all_tlens]
    num_blocks = sum(pages)
    gd = torch.Generator(device=device).manual_seed(seed + 1)
    query = torch.randn((ends[-1], hq, d), generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    key_cache = torch.randn((num_blocks, BLOCK_SIZE, hkv, d), generator=gd, device=device,
                            dtype=torch.float32).to(torch.bfloat16)
    perm = torch.randperm(num_blocks, generator=g)
    table = torch.zeros((total_rows, max(pages)), dtype=torch.int32)
    k = 0
    for b, p in enumerate(pages):
        table[b, :p] = perm[k:k + p].to(torch.int32)
        k += p
    table = table.to(device)
    lmax = max(tlens)
    raw_k = torch.randn((rows, lmax, hkv, d), generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    raw_v = torch.randn((rows, lmax, hkv, d), generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(d)
    # Exact LSE of each committed query over its scored prefix (fp32 matmul).
    lse = torch.zeros((ends[-1], hq), dtype=torch.float32, device=device)
    for b in range(rows):
        if counts[b] <= 0:
            continue
        qi = starts[b] + min(max(counts[b] - 1, 0), qlens[b] - 1)
        n = committed[b]
        dense = key_cache[table[b, : (n + BLOCK_SIZE - 1) // BLOCK_SIZE].long()].reshape(-1, hkv, d)[:n].float()
        qg = query[qi].float().reshape(hkv, hq // hkv, d)
        logits = torch.matmul(qg, dense.permute(1, 2, 0).contiguous()).reshape(hq, n) * scale
        lse[qi] = torch.logsumexp(logits, dim=-1)
    return dict(query=query, lse=lse, key_cache=key_cache, table=table, raw_k=raw_k, raw_v=raw_v, tlens=all_tlens,
                counts=counts + [0] * pad, starts=starts, qlens=qlens, committed=committed, slots=slots + [-1] * pad,
                rows=rows, total_rows=total_rows, scale=scale, lmax=lmax)


def algorithmic_bytes(spec, inp, plan_lens, active):
    """Bytes a perfect kernel must move (K read once; q, LSE, scores; selected K/V read + written; cos/sin)."""
    hq, hkv, d, chunk = spec["hq"], spec["hkv"], spec["d"], spec["chunk"]
    scored = [n for n, c in zip(inp["committed"], inp["counts"]) if c > 0]
    chunks = [(n + chunk - 1) // chunk for n in scored]
    score_bytes = sum(scored) * hkv * d * 2 + len(scored) * hq * (d * 2 + 4) + sum(chunks) * 4
    gathered = [h for h, a in zip(plan_lens, active) if a]
    gather_bytes = sum(gathered) * hkv * d * 2 * 4 + (max(gathered, default=0) * d * 2)
    chain_bytes = score_bytes + sum(chunks) * 4 + gather_bytes
    return score_bytes, gather_bytes, chain_bytes


def run(args):
    import torch

    from ds355 import _lib, step
    from ds355.plan import history_budget

    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1"}))
        log("bench.py measures one MI355X; runs over several GPUs are not supported")
        sys.exit(2)
    spec = WORKLOADS[args.workload]
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    lib = _lib.load()
    chunk, token_budget, d, hkv = spec["chunk"], spec["budget"], spec["d"], spec["hkv"]
    hb = history_budget(token_budget, DRAFT_TOKENS, chunk)
    t0 = time.time()
    copies = [build_inputs(spec, args.seed, device)]
    for _ in range(args.copies - 1):
        copies.append({k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in copies[0].items()})
    log(f"inputs ready in {time.time() - t0:.1f}s ({args.copies} copies)")
    inp0 = copies[0]
    total_rows, rows, lmax = inp0["total_rows"], inp0["rows"], inp0["lmax"]
    max_chunks = (max(inp0["tlens"]) + chunk - 1) // chunk
    inv = 1.0 / (ROPE_THETA ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.outer(torch.arange(token_budget, dtype=torch.float32), inv)
    cos_sin = torch.cat((freqs.cos(), freqs.sin()), -1).to(torch.bfloat16).to(device)
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=device)  # noqa: E731
    rows_t = dict(counts=i32(inp0["counts"]), starts=i32(inp0["starts"]), qlens=i32(inp0["qlens"]),
                  tlens=i32(inp0["tlens"]), slots=i32(inp0["slots"]), committed=i32(inp0["committed"]))
    g = torch.Generator().manual_seed(args.seed + 7)
    reuse = spec.get("reuse_half", False)
    active = [1] * total_rows
    if reuse:
        active = [int(x) for x in (torch.rand(total_rows, generator=g) >= 0.5)]
    row_active = i32(active) if reuse else None

    states = []
    for inp in copies:
        st = dict(
            scores=torch.zeros((total_rows, max_chunks), dtype=torch.float32, device=device),
            partials=torch.zeros((total_rows, max_chunks, hkv), dtype=torch.float32, device=device),
            sel_ids=torch.zeros((rows, token_budget // chunk), dtype=torch.int32, device=device),
            sel_count=torch.full((rows,), -1, dtype=torch.int32, device=device),
            plan=torch.zeros((total_rows, 5 + token_budget // chunk), dtype=torch.int64, device=device),
            working_lens=torch.zeros((rows,), dtype=torch.int32, device=device),
            work_k=torch.zeros((rows, hkv, token_budget, d), dtype=torch.bfloat16, device=device),
        )
        st["work_v"] = torch.zeros_like(st["work_k"])
        if args.path == "fused":
            st["workspace"] = step.new_workspace(total_rows, max_chunks, hkv, token_budget, device)
        states.append(st)

    descs = []
    for inp, st in zip(copies, states):
        desc, _ = step.build_step_desc(
            snapshot=step.VerifierSnapshot(inp["query"], inp["lse"], inp["key_cache"], inp["table"], inp["scale"]),
            rows=step.VerifierRows(rows_t["counts"], rows_t["starts"], rows_t["qlens"], rows_t["tlens"], rows),
            scores=st["scores"], score_partials=st["partials"], sel_ids=st["sel_ids"], sel_count=st["sel_count"], slots=rows_t["slots"],
            committed_lens=rows_t["committed"], plan=st["plan"], working_lens=st["working_lens"],
            raw_key=inp["raw_k"], raw_value=inp["raw_v"], working_key=st["work_k"], working_value=st["work_v"],
            cos_sin_cache=cos_sin, rotary_dim=d, is_neox_style=True, chunk_size=chunk, history_budget=hb,
            recent_window=spec.get("window", RECENT_WINDOW),
            row_active=row_active, workspace=st.get("workspace"),
        )
        descs.append(desc)
    stream = torch.cuda.current_stream(device).cuda_stream

    def launch(i, stages=None):
        desc = descs[i % len(descs)]
        if stages is not None:
            desc.stages = stages
        rc = lib.ds_retrieval_step(stream, desc)
        desc.stages = step.ALL
        if rc:
            _lib.check(rc)

    # A full step on every copy first: the plans the gather-only timing uses.
    for i in range(len(descs)):
        launch(i)
    torch.cuda.synchronize()
    # With a workspace the library runs the single launch when the batch
    # shape suits it (8+ rows) and the chain otherwise; the epochs tell which.
    single = False
    if args.path == "fused":
        epochs = [step.workspace_epoch(st["workspace"]) for st in states]
        single = epochs == [1] * len(states)
        if not single and any(epochs):
            raise RuntimeError(f"the single launch ran for some copies only (epochs {epochs})")

    # Untimed warmup, then exactly K timed steps bracketed by synchronisation.
    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    start.record()
    for i in range(args.steps):
        launch(i)
    stop.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t_wall) * 1e3
    chain_ms = start.elapsed_time(stop) / args.steps
    if single:
        # Every timed launch must have completed its waits: a launch whose
        # bounded wait expired leaves a status bit and invalid results.
        status = [step.workspace_status(st["workspace"]) for st in states]
        if any(status):
            raise RuntimeError(f"single-launch status words {status} after the timed steps: results not valid")

    # Per-kernel durations with HIP events on the launch stream.
    def time_stage(stages, reps):
        for i in range(3):
            launch(i, stages)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for i in range(reps):
            ev[i][0].record()
            launch(i, stages)
            ev[i][1].record()
        torch.cuda.synchronize()
        return statistics.mean(a.elapsed_time(b) for a, b in ev) * 1e3  # µs

    reps = max(20, args.steps // 2)
    step_us = time_stage(step.ALL, reps)
    score_us = time_stage(step.SCORE, reps)
    select_us = time_stage(step.SELECT, reps)
    # The runtime's retrieval call (SCORE | SELECT): one launch with a workspace.
    score_select_us = time_stage(step.SCORE | step.SELECT, reps)
    plan_gather_us = time_stage(step.PLAN, reps)

    # Gather alone through its C entry point (prebuilt arguments, so host
    # overhead stays below the kernel time), on the plans the chain produced.
    gather_args = []
    for inp, st in zip(copies, states):
        ra = None if row_active is None else row_active[:rows]
        gather_args.append((
            stream, _lib.DS_BF16, inp["raw_k"].data_ptr(), inp["raw_v"].data_ptr(), st["work_k"].data_ptr(),
            st["work_v"].data_ptr(), st["plan"].data_ptr(), rows, st["plan"].shape[1], cos_sin.data_ptr(),
            cos_sin.stride(0), cos_sin.shape[0], st["work_k"].shape[0], inp["raw_k"].shape[1], hkv, d, token_budget,
            chunk, d, 1, hb, None if ra is None else ra.data_ptr()))
    gather_ev = []
    for i in range(reps + 3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        _lib.check(lib.ds_rebuild_compact_kv(*gather_args[i % len(gather_args)]))
        b.record()
        gather_ev.append((a, b))
    torch.cuda.synchronize()
    gather_us = statistics.mean(a.elapsed_time(b) for a, b in gather_ev[3:]) * 1e3

    plan_lens = states[0]["plan"][:, 1].tolist()
    score_bytes, gather_bytes, chain_bytes = algorithmic_bytes(spec, inp0, plan_lens, active)
    score_gbps = score_bytes / (score_us * 1e-6) / 1e9
    gather_gbps = gather_bytes / (gather_us * 1e-6) / 1e9
    chain_gbps = chain_bytes / (chain_ms * 1e-3) / 1e9

    # Device copy bandwidth of a plain 1 GiB copy, for context.
    src = torch.empty(1 << 29, dtype=torch.int16, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(10):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    copy_gbps = 2 * src.numel() * 2 * 10 / (a.elapsed_time(b) * 1e-3) / 1e9
    del src, dst

    fused = single
    traffic = None
    traffic_file = ROOT / "profiles" / f"traffic_{args.workload}.json"
    if traffic_file.exists():
        key = "fused_kernel_hbm_bytes_per_launch" if fused else "score_kernel_hbm_bytes_per_launch"
        traffic = json.loads(traffic_file.read_text()).get(key)
    if fused:
        # The whole step is one kernel: it is the dominant (and only) one, and the
        # timed region is K back-to-back launches of it, so its average launch
        # duration is the timed region's average.
        roof_kernel, roof_bytes, roof_us = "fused_step_kernel", chain_bytes, chain_ms * 1e3
    else:
        roof_kernel, roof_bytes, roof_us = "chunk_score_kernel", score_bytes, score_us
    roof_gbps = roof_bytes / (roof_us * 1e-6) / 1e9

    # Scoring without a supplied LSE: the same pass stores each chunk's mass
    # per query head.  The full step runs as the single launch where the
    # supplied-LSE step does (its selectors merge the masses into the LSEs);
    # SCORE alone is the chain's pass plus lse_finalize_kernel.
    free_descs = []
    for inp, st in zip(copies, states):
        st["lse_partials"] = torch.zeros((total_rows, max_chunks, spec["hq"], 2), dtype=torch.float32, device=device)
        st["lse_out"] = torch.zeros((total_rows, spec["hq"]), dtype=torch.float32, device=device)
        desc, _ = step.build_step_desc(
            snapshot=step.VerifierSnapshot(inp["query"], None, inp["key_cache"], inp["table"], inp["scale"]),
            rows=step.VerifierRows(rows_t["counts"], rows_t["starts"], rows_t["qlens"], rows_t["tlens"], rows),
            scores=st["scores"], score_partials=st["partials"], sel_ids=st["sel_ids"], sel_count=st["sel_count"],
            slots=rows_t["slots"], committed_lens=rows_t["committed"], plan=st["plan"],
            working_lens=st["working_lens"], raw_key=inp["raw_k"], raw_value=inp["raw_v"], working_key=st["work_k"],
            working_value=st["work_v"], cos_sin_cache=cos_sin, rotary_dim=d, is_neox_style=True, chunk_size=chunk,
            history_budget=hb, recent_window=spec.get("window", RECENT_WINDOW), row_active=row_active,
            lse_partials=st["lse_partials"], lse_out=st["lse_out"], workspace=st.get("workspace"),
        )
        free_descs.append(desc)

    def time_free(stages, reps):
        def go(i):
            desc = free_descs[i % len(free_descs)]
            desc.stages = stages
            _lib.check(lib.ds_retrieval_step(stream, desc))
        for i in range(3):
            go(i)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for i in range(reps):
            ev[i][0].record()
            go(i)
            ev[i][1].record()
        torch.cuda.synchronize()
        return statistics.mean(a.elapsed_time(b) for a, b in ev) * 1e3  # µs

    free_score_us = time_free(step.SCORE, reps)
    free_epochs = [step.workspace_epoch(st["workspace"]) for st in states] if single else []
    free_step_events_us = time_free(step.ALL, reps)
    # The full step back to back, timed as `value` is (events only around the whole run).
    a_ev, b_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a_ev.record()
    for i in range(reps):
        desc = free_descs[i % len(free_descs)]
        desc.stages = step.ALL
        _lib.check(lib.ds_retrieval_step(stream, desc))
    b_ev.record()
    torch.cuda.synchronize()
    free_step_us = a_ev.elapsed_time(b_ev) * 1e3 / reps
    free_single = single and [step.workspace_epoch(st["workspace"]) for st in states] != free_epochs
    if free_single and any(step.workspace_status(st["workspace"]) for st in states):
        raise RuntimeError("a single launch without an LSE reported an expired wait: results not valid")
    free_gbps = score_bytes / (free_score_us * 1e-6) / 1e9
    lse_free_leg = {
        "what": "scores without a supplied softmax LSE: the scoring pass stores each chunk's mass per query "
                "head; the single launch's group workgroups (or, for SCORE alone and the chain, "
                "lse_finalize_kernel) merge them into each head's LSE and the chunk scores.  step_us: the full "
                "step back to back, timed as value is; score_us and step_us_events_per_launch put events "
                "around each launch",
        "score_us": round(free_score_us, 2), "step_us": round(free_step_us, 2),
        "step_us_events_per_launch": round(free_step_events_us, 2),
        "step_path": "single launch (fused_step_kernel)" if free_single else "chain",
        "step_us_with_lse": round(chain_ms * 1e3, 2),
        "score_us_with_lse": round(score_us, 2),
        "achieved_gbps": round(free_gbps, 1), "frac": round(free_gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes": score_bytes,
    }
    del free_descs
    for st in states:
        del st["lse_partials"], st["lse_out"]

    attention_leg = draft_attention_leg(spec, states, rows, hb, device, reps, args.seed, not args.no_cpu_baseline)
    capture_leg = draft_capture_leg(spec, copies, states, rows, device, reps, args.seed)
    host_leg = runtime_host_leg(spec, inp0, hb, device)

    cpu = None if args.no_cpu_baseline else cpu_baseline(spec, copies[0], cos_sin, hb, rows_t, active, reuse)
    if cpu is not None:
        cpu["gpu_speedup"] = round(cpu["value"] / (chain_ms * 1e3), 1)
    if single:
        status = [step.workspace_status(st["workspace"]) for st in states]
        if any(status):
            raise RuntimeError(f"single-launch status words {status} after the stage timings: results not valid")
    # The runtime's own path: its two calls (retrieval, then compact prefill),
    # with gather records as DiffSpecDraftCache keeps them.
    from ds355.runtime import SINGLE_LAUNCH_MIN_ROWS

    # The runtime's default: the final history rows move at retrieval when it runs as the single launch.
    runtime_step = runtime_path(copies, states, rows_t, rows, cos_sin, spec, hb, row_active, device, reps,
                                prefix=rows >= SINGLE_LAUNCH_MIN_ROWS)
    two_call_us = runtime_step["total_us"]
    runtime_step.update({
        "what": "DiffSpecDraftCache's calls per retrieval step, kernel time, as the runtime makes them by default: "
                "accept_target_queries (SCORE | SELECT, and PREFIX, every history row whose raw sources are final, "
                "when the retrieval runs as the single launch) and prepare_compact_prefill (PLAN with gather "
                "records); and a compact prefill between retrievals.  total_us and cycle_us_retrieval_every_4: "
                "the calls back to back, timed as the headline step is; the per-call times (and the "
                "*_events_per_call sums) put events around each call, which adds each launch's gap",
        "algorithmic_bytes": chain_bytes,
        "achieved_gbps": round(chain_bytes / (two_call_us * 1e-6) / 1e9, 1),
        "frac": round(chain_bytes / (two_call_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        "other_retrieval": runtime_path(copies, states, rows_t, rows, cos_sin, spec, hb, row_active, device,
                                               reps, prefix=rows < SINGLE_LAUNCH_MIN_ROWS),
        "without_records": runtime_path(copies, states, rows_t, rows, cos_sin, spec, hb, row_active, device, reps,
                                        records=False),
    })
    n_copies = len(copies)
    del copies, states, descs, gather_args
    torch.cuda.empty_cache()
    workloads = {}
    if not args.no_workloads:
        for name in WORKLOADS:
            if name == args.workload:
                continue
            log(f"workload {name}")
            workloads[name] = workload_leg(name, args.seed, device, with_cpu=not args.no_cpu_baseline)
        # The measured workload at two more seeds (other lengths, keys and page order).
        for extra in (0, 1, 2):
            if extra != args.seed:
                log(f"workload {args.workload} seed {extra}")
                workloads[f"{args.workload} seed {extra}"] = workload_leg(args.workload, extra, device, with_cpu=False)

    result = {
        "metric": METRIC,
        "value": round(chain_ms * 1e3, 2),
        "unit": "µs",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(chain_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload}: {rows} requests"
                        + (f" + {spec.get('pad')} padding rows" if spec.get("pad") else "")
                        + f", context {spec['lens']}, Hq {spec['hq']} / Hkv {hkv} x {d} bf16, chunk {chunk}, "
                          f"token budget {token_budget}, history {hb}, recent window "
                          f"{spec.get('window', RECENT_WINDOW)}, paged K block {BLOCK_SIZE}, "
                          f"{n_copies} rotated input copies",
            "global_batch": rows,
            "seq_len": max(inp0["tlens"]),
            "parallelism": "single GPU",
            "scored_tokens": sum(n for n, c in zip(inp0["committed"], inp0["counts"]) if c > 0),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": roof_kernel,
            "achieved": round(roof_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(roof_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes": roof_bytes,
            "avg_us": round(roof_us, 2),
        },
        "path": ("single launch (fused_step_kernel)" if fused else
                 "three-kernel chain" + (" (batch below the single launch's 8 rows)" if args.path == "fused" else "")),
        "kernels_us": {"step": round(step_us, 2), "chunk_score": round(score_us, 2), "select": round(select_us, 2),
                       "score_and_select": round(score_select_us, 2),
                       "plan_and_gather": round(plan_gather_us, 2), "gather": round(gather_us, 2)},
        "score_roofline": {"achieved": round(score_gbps, 1), "frac": round(score_gbps / HBM_PEAK_GBPS, 4),
                           "algorithmic_bytes": score_bytes},
        "gather_roofline": {"achieved": round(gather_gbps, 1), "frac": round(gather_gbps / HBM_PEAK_GBPS, 4),
                            "algorithmic_bytes": gather_bytes},
        "chain": {"algorithmic_bytes": chain_bytes, "achieved_gbps": round(chain_gbps, 1),
                  "frac": round(chain_gbps / HBM_PEAK_GBPS, 4), "wall_ms_total": round(wall_ms, 3)},
        "copy_gbps": round(copy_gbps, 1),
        "lse_free_scoring": lse_free_leg,
        "draft_attention": attention_leg,
        "draft_capture": capture_leg,
        "runtime_host": host_leg,
        "runtime_step": runtime_step,
        "workloads": workloads,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result, ensure_ascii=False), flush=True)


ATTENTION_COPIES = 6  # working caches rotated per launch: 6 x 67 MB exceeds the 256 MB MALL


def runtime_path(copies, states, rows_t, rows, cos_sin, spec, hb, row_active, device, reps, prefix=False,
                 records=True):
    """The plugin's own calls with gather records, as DiffSpecDraftCache makes
    them at the reference's cadence: a retrieval call (SCORE | SELECT; with
    ``prefix`` also each row's history prefix, one launch for 8+ rows) and
    the compact prefill after it (PLAN: plans and the gather of what the
    records do not hold), then the compact prefills of the three cycles up to
    the next retrieval, each at roots advanced by 0-4 tokens per row (the
    accepted drafts; seeded).  The selections stay; the rolling tail moves,
    and a row whose history prefix shifts (its prefix drop changes as the
    window slides over a selected chunk) moves whole.  HIP events around each
    launch, input copies rotated; per copy its own selection generations and
    records (``records=False``: the same calls without them, every compact
    prefill moving every row)."""
    import torch

    from ds355 import _lib, step

    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    chunk, token_budget, d = spec["chunk"], spec["budget"], spec["d"]
    pairs = []
    for c, st in zip(copies, states):
        held_state = (torch.zeros((rows,), dtype=torch.int32, device=device),
                      torch.zeros((rows, token_budget), dtype=torch.int64, device=device)) if records else None
        common = dict(
            sel_ids=st["sel_ids"], sel_count=st["sel_count"], slots=rows_t["slots"], plan=st["plan"],
            working_lens=st["working_lens"], raw_key=c["raw_k"], raw_value=c["raw_v"], working_key=st["work_k"],
            working_value=st["work_v"], cos_sin_cache=cos_sin, rotary_dim=d, is_neox_style=True, chunk_size=chunk,
            history_budget=hb, recent_window=spec.get("window", RECENT_WINDOW), row_active=row_active,
            gather_records=held_state)
        retrieve, _ = step.build_step_desc(
            stages=step.SCORE | step.SELECT | (step.PREFIX if prefix else 0),
            snapshot=step.VerifierSnapshot(c["query"], c["lse"], c["key_cache"], c["table"], c["scale"]),
            rows=step.VerifierRows(rows_t["counts"], rows_t["starts"], rows_t["qlens"], rows_t["tlens"], rows),
            scores=st["scores"], score_partials=st["partials"], committed_lens=None if prefix else rows_t["committed"],
            workspace=st.get("workspace") if prefix else None, **common)
        prefill, _ = step.build_step_desc(stages=step.PLAN, snapshot=None, rows=None, scores=None,
                                          committed_lens=rows_t["committed"], **common)
        pairs.append((retrieve, prefill, held_state))
    run = lambda desc: _lib.check(lib.ds_retrieval_step(stream, desc))  # noqa: E731
    epochs = [step.workspace_epoch(st["workspace"]) for st in states if "workspace" in st]
    for r, p, _ in pairs:
        run(r)
        run(p)
    torch.cuda.synchronize()
    single = bool(epochs) and [step.workspace_epoch(st["workspace"]) for st in states if "workspace" in st] != epochs
    # Roots of the three cycles after a retrieval: + 0-4 accepted tokens per cycle and row.
    g = torch.Generator().manual_seed(11)
    base = rows_t["committed"]
    step_len = torch.randint(0, DRAFT_TOKENS + 1, (base.numel(),), generator=g).to(base.device, base.dtype)
    roots = [base] + [base + k * step_len for k in (1, 2, 3)]
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(reps)]
    for i in range(reps):
        r, p, _ = pairs[i % len(pairs)]
        ev[i][0].record()
        run(r)
        for k, root in enumerate(roots):
            ev[i][k + 1].record()
            p.committed_lens = root.data_ptr()
            run(p)
        ev[i][5].record()
    torch.cuda.synchronize()
    # The same calls back to back, timed like the headline step (events only
    # around the whole sequence): the per-call events above add each launch's
    # gap.  The retrieval and its compact prefill, then the full four-cycle
    # sequence (retrieval, compact prefill, three compact prefills).
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(reps):
        r, p, _ = pairs[i % len(pairs)]
        run(r)
        p.committed_lens = base.data_ptr()
        run(p)
    b.record()
    torch.cuda.synchronize()
    pair_us = a.elapsed_time(b) * 1e3 / reps
    a.record()
    for i in range(reps):
        r, p, _ = pairs[i % len(pairs)]
        run(r)
        for root in roots:
            p.committed_lens = root.data_ptr()
            run(p)
    b.record()
    torch.cuda.synchronize()
    cycle4_us = a.elapsed_time(b) * 1e3 / reps
    for _, p, _ in pairs:
        p.committed_lens = base.data_ptr()
    retrieval_us = statistics.mean(e[0].elapsed_time(e[1]) for e in ev) * 1e3
    prefill_us = statistics.mean(e[1].elapsed_time(e[2]) for e in ev) * 1e3
    held_us = statistics.mean(e[k].elapsed_time(e[k + 1]) for e in ev for k in (2, 3, 4)) * 1e3
    if single and any(step.workspace_status(st["workspace"]) for st in states):
        raise RuntimeError("single-launch status words set after the retrieval calls: results not valid")
    held_tasks = sum(int((rec[1] != 0).sum()) for _, _, rec in pairs if rec is not None) // len(pairs)
    del pairs
    return {
        "retrieval_path": "single launch" if single else "chain", "final_rows_at_retrieval": bool(prefix),
        "total_us": round(pair_us, 2),
        "retrieval_us": round(retrieval_us, 2), "compact_prefill_us": round(prefill_us, 2),
        "total_us_events_per_call": round(retrieval_us + prefill_us, 2),
        "compact_prefill_between_retrievals_us": round(held_us, 2),
        "cycle_us_retrieval_every_4": round(cycle4_us / 4, 2),
        "cycle_us_retrieval_every_4_events_per_call": round((retrieval_us + prefill_us + 3 * held_us) / 4, 2),
        "held_tasks_per_copy": held_tasks,
        "roots_advance_per_cycle": "0-4 tokens per row (seeded)",
    }


def traffic_of(key, spec):
    """HBM bytes per launch measured with rocprofv3 PMC counters for this workload, if recorded."""
    name = next((k for k, v in WORKLOADS.items() if v is spec), None)
    path = ROOT / "profiles" / f"traffic_{name}.json"
    return json.loads(path.read_text()).get(key) if path.exists() else None


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def workload_leg(name, seed, device, steps=20, with_cpu=True):
    """One line per other configuration: the full step (single launch for
    8+ rows with a workspace, else the chain) timed back to back with HIP
    events over rotated input copies, its roofline fraction, the runtime's
    two calls (SCORE | SELECT, then the compact prefill) and the oracle's
    CPU step on a bounded sample of the same rows."""
    import torch

    from ds355 import _lib, step
    from ds355.plan import history_budget

    spec = WORKLOADS[name]
    chunk, token_budget, d, hkv = spec["chunk"], spec["budget"], spec["d"], spec["hkv"]
    hb = history_budget(token_budget, DRAFT_TOKENS, chunk)
    inp = build_inputs(spec, seed, device)
    rows, total_rows = inp["rows"], inp["total_rows"]
    scored = sum(n for n, c in zip(inp["committed"], inp["counts"]) if c > 0)
    step_bytes = scored * hkv * d * 2 + rows * hkv * hb * d * 2 * 4
    gather_bytes = sum(1 for b in range(rows) if not spec.get("reuse_half") or b % 2 == 0) * hkv * hb * d * 2 * 4
    # Enough rotated copies that neither the step nor the compact prefill
    # alone runs from a warm 256 MB MALL (at most 4).
    need = max(-(-(3 * MALL_BYTES // 2) // max(step_bytes, 1)), -(-(3 * MALL_BYTES // 2) // max(gather_bytes, 1)))
    copies = [inp]
    for _ in range(min(4, need) - 1):
        copies.append({k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()})
    max_chunks = (max(inp["tlens"]) + chunk - 1) // chunk
    inv = 1.0 / (ROPE_THETA ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.outer(torch.arange(token_budget, dtype=torch.float32), inv)
    cos_sin = torch.cat((freqs.cos(), freqs.sin()), -1).to(torch.bfloat16).to(device)
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32, device=device)  # noqa: E731
    rows_t = dict(counts=i32(inp["counts"]), starts=i32(inp["starts"]), qlens=i32(inp["qlens"]),
                  tlens=i32(inp["tlens"]), slots=i32(inp["slots"]), committed=i32(inp["committed"]))
    active = [1] * total_rows
    if spec.get("reuse_half"):
        g = torch.Generator().manual_seed(seed + 7)
        active = [int(x) for x in (torch.rand(total_rows, generator=g) >= 0.5)]
    row_active = i32(active) if spec.get("reuse_half") else None
    descs, keep = [], []
    for c in copies:
        st = dict(scores=torch.zeros((total_rows, max_chunks), dtype=torch.float32, device=device),
                  partials=torch.zeros((total_rows, max_chunks, hkv), dtype=torch.float32, device=device),
                  sel_ids=torch.zeros((rows, token_budget // chunk), dtype=torch.int32, device=device),
                  sel_count=torch.full((rows,), -1, dtype=torch.int32, device=device),
                  plan=torch.zeros((total_rows, 5 + token_budget // chunk), dtype=torch.int64, device=device),
                  working_lens=torch.zeros((rows,), dtype=torch.int32, device=device),
                  work_k=torch.zeros((rows, hkv, token_budget, d), dtype=torch.bfloat16, device=device),
                  workspace=step.new_workspace(total_rows, max_chunks, hkv, token_budget, device))
        st["work_v"] = torch.zeros_like(st["work_k"])
        desc, _ = step.build_step_desc(
            snapshot=step.VerifierSnapshot(c["query"], c["lse"], c["key_cache"], c["table"], c["scale"]),
            rows=step.VerifierRows(rows_t["counts"], rows_t["starts"], rows_t["qlens"], rows_t["tlens"], rows),
            scores=st["scores"], score_partials=st["partials"], sel_ids=st["sel_ids"], sel_count=st["sel_count"],
            slots=rows_t["slots"], committed_lens=rows_t["committed"], plan=st["plan"],
            working_lens=st["working_lens"], raw_key=c["raw_k"], raw_value=c["raw_v"], working_key=st["work_k"],
            working_value=st["work_v"], cos_sin_cache=cos_sin, rotary_dim=d, is_neox_style=True, chunk_size=chunk,
            history_budget=hb, recent_window=spec.get("window", RECENT_WINDOW), row_active=row_active,
            workspace=st["workspace"])
        descs.append(desc)
        keep.append(st)
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream

    def timed(stages, n):
        for i in range(3):
            descs[i % len(descs)].stages = stages
            _lib.check(lib.ds_retrieval_step(stream, descs[i % len(descs)]))
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(n):
            descs[i % len(descs)].stages = stages
            _lib.check(lib.ds_retrieval_step(stream, descs[i % len(descs)]))
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / n

    epochs0 = [step.workspace_epoch(st["workspace"]) for st in keep]
    step_us = timed(step.ALL, steps)
    single = [step.workspace_epoch(st["workspace"]) for st in keep] != epochs0
    status = [step.workspace_status(st["workspace"]) for st in keep]
    if any(status):
        raise RuntimeError(f"{name}: single-launch status words {status}: results not valid")
    plan_lens = keep[0]["plan"][:, 1].tolist()
    score_bytes, gather_bytes, chain_bytes = algorithmic_bytes(spec, inp, plan_lens, active)
    gbps = chain_bytes / (step_us * 1e-6) / 1e9
    from ds355.runtime import SINGLE_LAUNCH_MIN_ROWS

    rt = runtime_path(copies, keep, rows_t, rows, cos_sin, spec, hb, row_active, device, max(10, steps // 2),
                      prefix=rows >= SINGLE_LAUNCH_MIN_ROWS)
    two_call = rt["total_us"]
    leg = {
        "config": f"{rows} requests" + (f" + {spec['pad']} padding rows" if spec.get("pad") else "")
                  + f", context {spec['lens']}, Hq {spec['hq']} / Hkv {hkv} x {d}, chunk {chunk}, token budget "
                    f"{token_budget}, history {hb}, window {spec.get('window', RECENT_WINDOW)}"
                  + (", half the rows keep their working rows" if spec.get("reuse_half") else ""),
        "seed": seed,
        "scored_tokens": sum(n for n, c in zip(inp["committed"], inp["counts"]) if c > 0),
        "path": "single launch" if single else "chain",
        "step_us": round(step_us, 2),
        "algorithmic_bytes": chain_bytes,
        "achieved_gbps": round(gbps, 1),
        "frac": round(gbps / HBM_PEAK_GBPS, 4),
        "mall": (f"step {'cold' if step_bytes * len(copies) > MALL_BYTES else 'warm'}, compact prefill "
                 f"{'cold' if gather_bytes * len(copies) > MALL_BYTES else 'warm'} ({len(copies)} rotated copies "
                 f"of {step_bytes / 1e6:.0f} MB and {gather_bytes / 1e6:.0f} MB against the 256 MB MALL)"),
        "copies": len(copies),
        "runtime_two_calls_us": dict(rt, frac=round(chain_bytes / (two_call * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                                     other_retrieval=runtime_path(copies, keep, rows_t, rows, cos_sin, spec, hb,
                                                                  row_active, device, max(10, steps // 2),
                                                                  prefix=rows < SINGLE_LAUNCH_MIN_ROWS),
                                     without_records=runtime_path(copies, keep, rows_t, rows, cos_sin, spec, hb,
                                                                  row_active, device, max(10, steps // 2),
                                                                  records=False)),
    }
    if with_cpu:
        leg["cpu_baseline"] = cpu_sample(spec, inp, cos_sin, hb, active)
    del descs, keep, copies, inp
    torch.cuda.empty_cache()
    return leg


def cpu_sample(spec, inp, cos_sin, hb, active, max_rows=4):
    """The oracle's CPU step on the first few committed rows of a workload
    (their pages, query, LSE and raw rows copied to the host), median of 3
    after 1 warm-up, on all host threads."""
    import torch

    from oracle import diffspec_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    chunk, token_budget, d = spec["chunk"], spec["budget"], spec["d"]
    ends = [s + q for s, q in zip(inp["starts"], inp["qlens"])]
    rows_idx, q_index, lengths = O.retrieval_rows(inp["counts"], ends, inp["tlens"], inp["rows"])
    rows_idx, q_index, lengths = rows_idx[:max_rows], q_index[:max_rows], lengths[:max_rows]
    bs = inp["key_cache"].shape[1]
    pages = [(n + bs - 1) // bs for n in lengths]
    table = torch.zeros((len(rows_idx), max(pages)), dtype=torch.int32)
    blocks, k = [], 0
    for j, b in enumerate(rows_idx):
        blocks.append(inp["table"][b, : pages[j]].long())
        table[j, : pages[j]] = torch.arange(k, k + pages[j], dtype=torch.int32)
        k += pages[j]
    key_cache = inp["key_cache"][torch.cat(blocks)].cpu()
    slots = [inp["slots"][b] for b in rows_idx]
    raw_k = inp["raw_k"][slots].cpu()
    raw_v = inp["raw_v"][slots].cpu()
    query = inp["query"][q_index].cpu()
    lse = inp["lse"][q_index].cpu()
    work_k = torch.zeros((len(rows_idx), spec["hkv"], token_budget, d), dtype=torch.bfloat16)
    work_v = torch.zeros_like(work_k)
    hist_ends = [max(0, inp["committed"][b] - 1) for b in rows_idx]
    regather = [bool(active[b]) for b in rows_idx] if spec.get("reuse_half") else None
    cs = cos_sin.cpu()

    def one():
        O.retrieval_step(query, lse, key_cache, table, lengths, raw_k, raw_v, work_k, work_v,
                         list(range(len(rows_idx))), hist_ends, cs, chunk_size=chunk, budget=hb,
                         token_budget=token_budget, scale=inp["scale"], rotary_dim=d, is_neox_style=True,
                         regather=regather, recent_window=spec.get("window", RECENT_WINDOW))

    one()
    times = []
    for _ in range(3):
        t = time.perf_counter()
        one()
        times.append(time.perf_counter() - t)
    return {"value": round(statistics.median(times) * 1e6, 1), "unit": "µs", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"the oracle's step on {len(rows_idx)} of the workload's committed rows "
                                      f"({sum(lengths)} scored tokens), median of 3 after 1 warm-up"}


def draft_attention_leg(spec, states, rows, hb, device, reps, seed, with_cpu):
    """Linear draft attention (one launch of draft_attention_kernel) over the
    working caches the step just gathered: every row at the K draft steps'
    local positions hb, hb + 1, ... in turn (the root token attends at the
    history length, each draft token one further)."""
    import torch

    from ds355 import _lib, attention

    hq, hkv, d, budget = spec["hq"], spec["hkv"], spec["d"], spec["budget"]
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator().manual_seed(seed + 11)
    slots = torch.arange(rows, dtype=torch.int32, device=device)
    positions = [torch.full((rows,), hb + s, dtype=torch.int32, device=device) for s in range(DRAFT_TOKENS)]
    sets = []
    for i in range(ATTENTION_COPIES):
        st = states[i % len(states)]
        wk = st["work_k"] if i < len(states) else st["work_k"].clone()
        wv = st["work_v"] if i < len(states) else st["work_v"].clone()
        q = torch.randn((rows, hq, d), generator=g).to(torch.bfloat16).to(device)
        k = torch.randn((rows, hkv, d), generator=g).to(torch.bfloat16).to(device)
        v = torch.randn((rows, hkv, d), generator=g).to(torch.bfloat16).to(device)
        sets.append(dict(q=q, k=k, v=v, out=torch.empty_like(q), wk=wk, wv=wv,
                         lens=torch.zeros((rows,), dtype=torch.int32, device=device),
                         ws=attention.new_attention_workspace(rows, hq, hkv, d, budget, device)))
    calls = []
    for i in range(ATTENTION_COPIES * DRAFT_TOKENS):
        t = sets[i % ATTENTION_COPIES]
        calls.append((stream, _lib.DS_BF16, t["q"].data_ptr(), hq * d, d, t["k"].data_ptr(), hkv * d, d,
                      t["v"].data_ptr(), hkv * d, d, t["out"].data_ptr(), hq * d, d, t["wk"].data_ptr(),
                      t["wv"].data_ptr(), t["lens"].data_ptr(), slots.data_ptr(),
                      positions[(i // ATTENTION_COPIES) % DRAFT_TOKENS].data_ptr(), rows, rows, rows, hq, hkv, d,
                      budget, d ** -0.5, t["ws"].data_ptr(), t["ws"].numel()))
    for c in calls:
        _lib.check(lib.ds_draft_attention(*c))
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for i in range(reps):
        ev[i][0].record()
        _lib.check(lib.ds_draft_attention(*calls[i % len(calls)]))
        ev[i][1].record()
    torch.cuda.synchronize()
    avg_us = statistics.mean(a.elapsed_time(b) for a, b in ev) * 1e3
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(reps):
        _lib.check(lib.ds_draft_attention(*calls[i % len(calls)]))
    b.record()
    torch.cuda.synchronize()
    back_to_back_us = a.elapsed_time(b) * 1e3 / reps
    # A draft cycle's pattern: K steps over the same working caches (67 MB at
    # 16 rows), which stay in the 256 MB MALL between the steps.
    one = [c for i, c in enumerate(calls) if i % ATTENTION_COPIES == 0]
    for c in one:
        _lib.check(lib.ds_draft_attention(*c))
    torch.cuda.synchronize()
    a.record()
    for i in range(reps):
        _lib.check(lib.ds_draft_attention(*one[i % len(one)]))
    b.record()
    torch.cuda.synchronize()
    one_cache_us = a.elapsed_time(b) * 1e3 / reps
    status = [attention.attention_status(t["ws"]) for t in sets]
    if any(status):
        raise RuntimeError(f"draft attention status words {status}")
    mean_n = hb + (DRAFT_TOKENS + 1) / 2  # positions hb .. hb + K - 1 -> lengths hb + 1 .. hb + K
    kv_bytes = rows * mean_n * hkv * d * 2 * 2
    io_bytes = rows * hq * d * 2 * 2 + rows * hkv * d * 2 * 2  # q in, out, new K/V rows written
    algo = int(kv_bytes + io_bytes)
    # Back-to-back launches give the kernel's own duration (what a kernel
    # trace reports); events around each launch add the launch latency.
    gbps = algo / (back_to_back_us * 1e-6) / 1e9
    leg = {
        "workload": f"{rows} rows at local positions {hb}..{hb + DRAFT_TOKENS - 1} over the gathered working "
                    f"caches [rows, {hkv}, {budget}, {d}] bf16, Hq {hq}, {ATTENTION_COPIES} rotated copies",
        "kernel": "draft_attention_kernel",
        "avg_us": round(back_to_back_us, 2),
        "single_launch_event_us": round(avg_us, 2),
        "one_cache_us": round(one_cache_us, 2),
        "algorithmic_bytes": algo,
        "achieved": round(gbps, 1),
        "peak": HBM_PEAK_GBPS,
        "frac": round(gbps / HBM_PEAK_GBPS, 4),
        "traffic": traffic_of("attention_kernel_hbm_bytes_per_launch", spec),
    }
    if with_cpu:  # the oracle timed on the host cores, as the step's cpu_baseline is
        from oracle import diffspec_oracle as oracle

        t = sets[0]
        cpu_q, cpu_k, cpu_v = t["q"].cpu(), t["k"].cpu(), t["v"].cpu()
        cpu_wk, cpu_wv = t["wk"].cpu(), t["wv"].cpu()
        out = torch.empty_like(cpu_q)
        times = []
        for _ in range(4):
            lens = [0] * rows
            started = time.perf_counter()
            oracle.draft_linear_attention(cpu_q, cpu_k, cpu_v, d ** -0.5, out, cpu_wk, cpu_wv, lens,
                                          list(range(rows)), [hb] * rows)
            times.append(time.perf_counter() - started)
        leg["cpu_oracle_us"] = round(statistics.median(times[1:]) * 1e6, 1)
        leg["cpu_threads"] = torch.get_num_threads()
    return leg


def draft_capture_leg(spec, copies, states, rows, device, reps, seed):
    """Raw pre-RoPE K/V capture of one draft token per row plus the RoPE input
    (one launch of capture_kernel): each row's token at its last committed
    position, local positions from the working lengths the step just wrote."""
    import torch

    from ds355 import _lib

    hkv, d = spec["hkv"], spec["d"]
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator().manual_seed(seed + 13)
    slots = torch.arange(rows, dtype=torch.int32, device=device)
    rope = torch.zeros((rows * 64,), dtype=torch.int64, device=device)
    calls = []
    keep = []
    for inp, st in zip(copies, states):
        key = torch.randn((rows, hkv * d), generator=g).to(torch.bfloat16).to(device)
        value = torch.randn((rows, hkv * d), generator=g).to(torch.bfloat16).to(device)
        # the last committed position of each row (always inside the raw cache)
        positions = torch.tensor([max(c - 1, 0) for c in inp["committed"][:rows]], dtype=torch.int64, device=device)
        keep += [key, value, positions]
        calls.append((stream, _lib.DS_BF16, key.data_ptr(), hkv * d, d, value.data_ptr(), hkv * d, d,
                      positions.data_ptr(), 1, slots.data_ptr(), rows, inp["raw_k"].data_ptr(),
                      inp["raw_v"].data_ptr(), inp["raw_k"].shape[0], inp["raw_k"].shape[1], hkv, d,
                      st["working_lens"].data_ptr(), None, rope.data_ptr(), rows, rows, None))
    for c in calls:
        _lib.check(lib.ds_capture_raw_kv(*c))
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(reps):
        _lib.check(lib.ds_capture_raw_kv(*calls[i % len(calls)]))
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / reps
    moved = rows * hkv * d * 2 * 2 * 2 + rows * (4 + 8 + 4 + 8)  # K/V rows in and out; slots, positions, lens, RoPE
    return {
        "workload": f"{rows} rows, one draft token each, K/V [{rows}, {hkv}x{d}] bf16 into the raw caches, "
                    f"int64 positions, local positions from working_lens",
        "kernel": "capture_kernel",
        "avg_us": round(us, 2),
        "algorithmic_bytes": moved,
        "note": "one launch per draft step; the reference builds index tensors on the host and runs torch index ops",
    }


def runtime_host_leg(spec, inp, hb, device, cycles=40):
    """Host time of DiffSpecDraftCache's calls over whole draft cycles.

    One cycle: verifier snapshot, retrieval (SCORE | SELECT), draft cycle
    start, compact prefill (PLAN), then K = 4 draft steps of raw-KV capture
    and draft attention.  Each call is timed on the host without a
    synchronisation (launches are asynchronous); the cycle time ends with
    one.  Medians after 5 warm-up cycles, in µs.
    """
    import torch

    from ds355 import runtime

    rows, hkv, d, hq = inp["rows"], spec["hkv"], spec["d"], spec["hq"]

    class Rotary:
        rotary_dim = d
        is_neox_style = True

    inv = 1.0 / (ROPE_THETA ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.outer(torch.arange(spec["budget"], dtype=torch.float32), inv)
    rotary = Rotary()
    rotary.cos_sin_cache = torch.cat((freqs.cos(), freqs.sin()), -1).to(torch.bfloat16).to(device)
    settings = runtime.DiffSpecSettings(chunk_size=spec["chunk"], token_budget=spec["budget"], retrieval_interval=1,
                                        max_tree_nodes=4, max_tree_depth=DRAFT_TOKENS, tree_threshold=0.7,
                                        adaptive_profile=False, recent_window=spec.get("window", RECENT_WINDOW))
    cache = runtime.DiffSpecDraftCache(settings, max_num_reqs=rows, max_model_len=inp["lmax"], num_kv_heads=hkv,
                                       head_dim=d, target_num_layers=2, dtype=torch.bfloat16, device=device,
                                       rotary_embedding=rotary)
    ids = [f"request-{i}" for i in range(rows)]
    ends = [s + q for s, q in zip(inp["starts"], inp["qlens"])][:rows]
    meta = types.SimpleNamespace(actual_seq_lengths_q=ends, seq_lens_list=inp["tlens"][:rows],
                                 block_tables=inp["table"][:rows], num_prefills=0)
    counts = torch.tensor(inp["counts"][:rows], dtype=torch.int32, device=device)
    g = torch.Generator(device=device).manual_seed(5)
    q = torch.randn((rows, hq, d), generator=g, device=device).to(torch.bfloat16)
    k = torch.randn((rows, hkv * d), generator=g, device=device).to(torch.bfloat16)
    v = torch.randn((rows, hkv, d), generator=g, device=device).to(torch.bfloat16)
    out = torch.empty((rows, hq * d), dtype=torch.bfloat16, device=device)
    pos = torch.tensor([max(c - 1, 0) for c in inp["committed"][:rows]], dtype=torch.int64, device=device)
    names = ("capture_target_attention", "accept_target_queries", "prepare_compact_prefill", "capture_raw_kv",
             "forward_attention", "cycle_issue", "cycle")
    times = {n: [] for n in names}

    def timed(name, fn):
        t = time.perf_counter()
        fn()
        times[name].append((time.perf_counter() - t) * 1e6)

    for it in range(cycles + 5):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cache.begin_target_forward(ids)
        timed("capture_target_attention", lambda: cache.capture_target_attention(
            inp["query"][: ends[-1]], inp["lse"][: ends[-1]], inp["key_cache"], meta, inp["scale"]))
        timed("accept_target_queries", lambda: cache.accept_target_queries(counts, is_prefill=False))
        cache.begin_cycle(ids)
        timed("prepare_compact_prefill", lambda: cache.prepare_compact_prefill(
            meta, rows, committed_seq_lens=inp["committed"][:rows]))
        for step_i in range(DRAFT_TOKENS):
            if step_i:
                cache.prepare_draft_step()
            timed("capture_raw_kv", lambda: cache.capture_raw_kv(0, pos + step_i, k, v))
            timed("forward_attention", lambda: cache.forward_attention(q, k, v, inp["scale"], out))
        cache.end_cycle()
        times["cycle_issue"].append((time.perf_counter() - t0) * 1e6)
        torch.cuda.synchronize()
        times["cycle"].append((time.perf_counter() - t0) * 1e6)
        if it == 4:
            for n in names:
                times[n].clear()
    result = {n: round(statistics.median(xs), 1) for n, xs in times.items()}
    del cache
    return {
        "what": f"host µs per DiffSpecDraftCache call, median over {cycles} draft cycles of {rows} requests "
                f"(retrieval, compact prefill, {DRAFT_TOKENS} draft steps); 'cycle_issue' is the host time to "
                f"issue a whole cycle, 'cycle' its wall time ending with one synchronisation",
        **result,
    }


def cpu_baseline(spec, inp, cos_sin, hb, rows_t, active, reuse):
    """The oracle's CPU restatement of the reference path, timed on this host."""
    import torch

    from oracle import diffspec_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    chunk, token_budget, d = spec["chunk"], spec["budget"], spec["d"]
    rows = inp["rows"]
    t0 = time.time()
    real = [b for b in range(inp["total_rows"]) if inp["counts"][b] > 0]
    _, q_index, lengths = O.retrieval_rows(inp["counts"], [s + q for s, q in zip(inp["starts"], inp["qlens"])],
                                           inp["tlens"], rows)
    query = inp["query"][q_index].cpu()
    lse = inp["lse"][q_index].cpu()
    key_cache = inp["key_cache"].cpu()
    table = inp["table"][real].cpu()
    raw_k, raw_v = inp["raw_k"].cpu(), inp["raw_v"].cpu()
    work_k = torch.zeros((rows, spec["hkv"], token_budget, d), dtype=torch.bfloat16)
    work_v = torch.zeros_like(work_k)
    cs = cos_sin.cpu()
    slots = [inp["slots"][b] for b in real]
    ends = [max(0, inp["committed"][b] - 1) for b in real]
    regather = [bool(active[b]) for b in real] if reuse else None
    log(f"cpu baseline inputs copied in {time.time() - t0:.1f}s")

    def one():
        O.retrieval_step(query, lse, key_cache, table, lengths, raw_k, raw_v, work_k, work_v, slots, ends, cs,
                         chunk_size=chunk, budget=hb, token_budget=token_budget, scale=inp["scale"], rotary_dim=d,
                         is_neox_style=True, regather=regather, recent_window=spec.get("window", RECENT_WINDOW))

    t = time.perf_counter()
    one()  # warm-up
    first = time.perf_counter() - t
    reps = max(1, min(5, int(20.0 / max(first, 1e-3))))
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        one()
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    cpu_model = platform.processor() or ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(med * 1e6, 1),
        "unit": "µs",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"the full step ({len(real)} requests, same inputs), median of {reps} runs after 1 warm-up; "
                  f"os.cpu_count()={os.cpu_count()}, cpu='{cpu_model}'",
        "gpu_speedup": None,
    }


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    parser.add_argument("--copies", type=int, default=3, help="rotated input copies (defeats the 256 MB MALL)")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-workloads", action="store_true", help="skip the other configurations' lines")
    parser.add_argument("--path", choices=("fused", "chain"), default="fused",
                        help="fused: the single-launch step (default); chain: the three-kernel chain")
    args = parser.parse_args()
    run(args)


if __name__ == "__main__":
    main()
