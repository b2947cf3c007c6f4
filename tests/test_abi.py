"""C-ABI checks that need no GPU: exports, struct layout, validation, no CPU fallback."""

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ds355.h"


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ds_[a-z_0-9]+)\s*\(", text)))


def _step_desc_fields():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct ds_step_desc \{(.*?)\} ds_step_desc;", text, flags=re.S).group(1)
    fields = []
    for decl in body.split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        m = re.match(r"(const )?(int64_t|uint64_t|int32_t|int|float|void|size_t)\s*(\*?)\s*(.*)", decl)
        assert m, decl
        kind = "ptr" if m.group(3) else m.group(2)
        for name in m.group(4).split(","):
            fields.append((name.strip().lstrip("*").strip(), kind))
    return fields


def test_library_exports_every_declared_symbol():
    from ds355 import _lib

    lib = _lib.load()
    declared = _declared_functions()
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.ds_abi_version() == _lib.ABI_VERSION
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", str(_lib.LIBRARY_PATH)], capture_output=True, text=True)
        exported = set(re.findall(r" T (ds_[a-z_0-9]+)", out.stdout))
        assert exported == set(declared)


def test_step_desc_matches_header_fields():
    from ds355 import _lib

    sizes = {"ptr": ctypes.c_void_p, "int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float,
             "int32_t": ctypes.c_int32, "size_t": ctypes.c_size_t}
    header = _step_desc_fields()
    py = [(name, t) for name, t in _lib.StepDesc._fields_]
    assert [n for n, _ in header] == [n for n, _ in py]
    for (name, kind), (_, ctype) in zip(header, py):
        assert ctypes.sizeof(sizes[kind]) == ctypes.sizeof(ctype), name


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_step_desc_offsets_match_c_compiler(tmp_path):
    from ds355 import _lib

    names = [n for n, _ in _lib.StepDesc._fields_]
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {",
             '  printf("%zu\\n", sizeof(ds_step_desc));']
    lines += [f'  printf("%zu\\n", offsetof(ds_step_desc, {n}));' for n in names]
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-O0", "-o", str(exe), str(src)], check=True)
    values = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert values[0] == ctypes.sizeof(_lib.StepDesc)
    for name, offset in zip(names, values[1:]):
        assert getattr(_lib.StepDesc, name).offset == offset, name


def test_c_side_validation_reports_reference_messages():
    """Argument checks run before any HIP call, so they are exercised without a GPU."""
    from ds355 import _lib

    lib = _lib.load()
    rc = lib.ds_rebuild_compact_kv(None, _lib.DS_BF16, None, None, None, None, None, 1, 9, None, 16, 8,
                                   2, 8, 1, 16, 8, 2, 3, 1, 4, None)
    assert rc == _lib.DS_ERR_INVALID
    assert lib.ds_last_error().decode() == "rotary_dim must be even and between zero and head_dim"
    rc = lib.ds_rebuild_compact_kv(None, _lib.DS_BF16, None, None, None, None, None, 1, 8, None, 16, 8,
                                   2, 8, 1, 16, 8, 2, 16, 1, 4, None)
    assert rc == _lib.DS_ERR_INVALID
    assert lib.ds_last_error().decode() == "plan width must be 5 + working_budget // chunk_size"
    rc = lib.ds_chunk_scores(None, _lib.DS_BF16, None, 0, None, 0, 0, 0, None, 0, 0, None, 0, None,
                             1, 6, 4, 128, 16, 64, 1, 1.0, 0, None, 0, None, 0)
    assert rc == _lib.DS_ERR_INVALID
    assert lib.ds_last_error().decode() == "query heads must be divisible by KV heads"
    rc = lib.ds_chunk_scores(None, _lib.DS_BF16, None, 0, None, 0, 0, 0, None, 0, 0, None, 0, None,
                             1, 64, 2, 128, 16, 64, 1, 1.0, 0, None, 0, None, 0)
    assert rc == _lib.DS_ERR_UNSUPPORTED
    rc = lib.ds_select_chunks(None, None, 4, 4, None, 1, 4, 6, None, 4, None)
    assert rc == _lib.DS_ERR_INVALID
    assert lib.ds_last_error().decode() == "token_budget must be a positive chunk-size multiple"
    desc = _lib.StepDesc()
    desc.stages = 16
    assert lib.ds_retrieval_step(None, desc) == _lib.DS_ERR_INVALID
    assert "unknown stage bits" in lib.ds_last_error().decode()
    # The prefix stage needs gather records, and the selection in the same call.
    desc.stages = _lib.DS_STAGE_PREFIX
    assert lib.ds_retrieval_step(None, desc) == _lib.DS_ERR_INVALID
    assert "needs gather records" in lib.ds_last_error().decode()
    desc.sel_gen, desc.gather_rec, desc.rec_stride = 64, 64, 1 << 20  # never dereferenced: refused first
    assert lib.ds_retrieval_step(None, desc) == _lib.DS_ERR_INVALID
    assert "runs with DS_STAGE_SELECT" in lib.ds_last_error().decode()
    desc.gather_rec = None
    desc.stages = _lib.DS_STAGE_PLAN
    assert lib.ds_retrieval_step(None, desc) == _lib.DS_ERR_INVALID
    assert "come together" in lib.ds_last_error().decode()


def test_lse_free_validation_without_gpu():
    """Scoring without an LSE: workspace sizing, the head-mean restriction and the step's pair buffer.

    The pointers are placeholders: every call fails its argument checks before
    any HIP call or launch.
    """
    from ds355 import _lib

    lib = _lib.load()
    fake = 1 << 12  # 16-byte aligned, never dereferenced
    # batch 2, Hq 8, Hkv 2, 3 chunks: (2 + 2 * 8) floats per (row, chunk) and 8 LSEs per row.
    need = 2 * (3 * (2 + 2 * 8) + 8) * 4
    args = [None, _lib.DS_BF16, fake, 8 * 128, fake, 16 * 2 * 128, 2 * 128, 128, None, 0, 0, fake, 4, fake,
            2, 8, 2, 128, 16, 64, 3, 1.0, _lib.DS_HEAD_MEAN, fake, 3]
    rc = lib.ds_chunk_scores(*args, fake, 2 * 3 * 2 * 4)  # room for the partials only
    assert rc == _lib.DS_ERR_INVALID
    assert lib.ds_last_error().decode() == (
        f"workspace too small: need {need} bytes without an LSE "
        "(batch * (max_chunks * (kv_heads + 2 * q_heads) + q_heads) * 4)")
    args[22] = _lib.DS_HEAD_MAX
    assert lib.ds_chunk_scores(*args, fake, need) == _lib.DS_ERR_UNSUPPORTED
    assert lib.ds_last_error().decode() == "head_reduce=max needs a supplied softmax LSE"

    desc = _lib.StepDesc()
    desc.stages = _lib.DS_STAGE_SCORE
    desc.batch_rows = desc.batch_size = 1
    desc.chunk_size, desc.history_budget, desc.token_budget = 64, 128, 256
    desc.plan_width, desc.sel_stride = 5 + 4, 4
    desc.counts = desc.query_start = desc.query_len = desc.target_len = fake
    desc.max_chunks, desc.scores, desc.score_partials = 4, fake, fake
    desc.num_kv_heads, desc.num_q_heads = 2, 8
    assert lib.ds_retrieval_step(None, desc) == _lib.DS_ERR_INVALID
    msg = ("without a softmax LSE the step needs lse_partials ([batch_rows, max_chunks, Hq, 2] fp32) and "
           "lse_out ([batch_rows, Hq] fp32)")
    assert lib.ds_last_error().decode() == msg
    desc.lse_partials = fake  # the LSE output is required too
    assert lib.ds_retrieval_step(None, desc) == _lib.DS_ERR_INVALID
    assert lib.ds_last_error().decode() == msg
    # ... with room for every query head per row, checked before anything is launched.
    desc.lse_out, desc.lse_out_stride = fake, 4
    desc.query = desc.key_cache = desc.block_table = fake
    desc.block_size, desc.head_dim = 16, 128
    assert lib.ds_retrieval_step(None, desc) == _lib.DS_ERR_INVALID
    assert lib.ds_last_error().decode() == "LSE output rows must hold every query head"


def test_lse_free_host_checks():
    """The Python wrappers refuse the LSE-free variant where it is not defined."""
    from ds355 import step
    from ds355.kernels import paged_chunk_attention_scores

    q = torch.zeros((1, 4, 32), dtype=torch.bfloat16)
    k = torch.zeros((2, 16, 1, 32), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="needs a supplied softmax_lse"):
        paged_chunk_attention_scores(q, k, None, torch.zeros((1, 2), dtype=torch.int32),
                                     torch.ones(1, dtype=torch.int32), chunk_size=4, max_seq_len=4, scale=1.0,
                                     head_reduce="max")
    with pytest.raises(ValueError, match="GPU only"):
        paged_chunk_attention_scores(q, k, None, torch.zeros((1, 2), dtype=torch.int32),
                                     torch.ones(1, dtype=torch.int32), chunk_size=4, max_seq_len=4, scale=1.0)
    i32 = lambda *s: torch.zeros(s, dtype=torch.int32)  # noqa: E731
    raw = torch.zeros((2, 64, 1, 32), dtype=torch.bfloat16)
    work = torch.zeros((2, 1, 32, 32), dtype=torch.bfloat16)
    common = dict(
        snapshot=step.VerifierSnapshot(q, None, k, i32(1, 2), 1.0),
        rows=step.VerifierRows(i32(1), i32(1), i32(1), i32(1), 1),
        scores=torch.zeros((1, 4)), score_partials=torch.zeros((1, 4, 1)), sel_ids=i32(2, 4), sel_count=i32(2),
        slots=i32(1), committed_lens=i32(1), plan=torch.zeros((1, 9), dtype=torch.int64), working_lens=None,
        raw_key=raw, raw_value=raw, working_key=work, working_value=work,
        cos_sin_cache=torch.zeros((64, 32), dtype=torch.bfloat16), rotary_dim=32, is_neox_style=True,
        chunk_size=4, history_budget=16,
    )
    with pytest.raises(ValueError, match="lse_partials must be a contiguous fp32"):
        step.build_step_desc(**common)
    for bad in (None, torch.zeros((1, 3))):
        with pytest.raises(ValueError, match="lse_out must be fp32"):
            step.build_step_desc(**common, lse_partials=torch.zeros((1, 4, 4, 2)), lse_out=bad)
    with pytest.raises(ValueError, match="GPU only"):
        step.build_step_desc(**common, lse_partials=torch.zeros((1, 4, 4, 2)), lse_out=torch.zeros((1, 4)))


def test_no_cpu_fallback():
    """Every product entry point refuses CPU tensors instead of computing on the host."""
    from ds355.compact_kv import rebuild_compact_kv_from_plan
    from ds355.kernels import paged_chunk_attention_scores
    from ds355.selection import select_context_chunks

    q = torch.zeros((1, 4, 32), dtype=torch.bfloat16)
    k = torch.zeros((2, 16, 1, 32), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        paged_chunk_attention_scores(q, k, torch.zeros(4), torch.zeros((1, 2), dtype=torch.int32),
                                     torch.ones(1, dtype=torch.int32), chunk_size=4, max_seq_len=4, scale=1.0)
    with pytest.raises(ValueError, match="GPU only"):
        select_context_chunks(torch.rand(4), 16, 4, 8)
    raw = torch.zeros((2, 8, 1, 32), dtype=torch.bfloat16)
    work = torch.zeros((2, 1, 8, 32), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        rebuild_compact_kv_from_plan(raw, raw, work, work, torch.zeros((1, 9), dtype=torch.int64),
                                     torch.zeros((8, 32), dtype=torch.bfloat16), chunk_size=2, max_width=2,
                                     rotary_dim=32, is_neox_style=True)


def test_reference_validation_order_on_host():
    """The drop-in wrappers raise the reference's messages before touching the device."""
    from ds355.compact_kv import rebuild_compact_kv_from_plan
    from ds355.kernels import paged_chunk_attention_scores

    with pytest.raises(ValueError, match=r"query must have shape \[batch, query_heads, head_dim\]"):
        paged_chunk_attention_scores(torch.zeros(4, 32), torch.zeros(1, 1, 1, 32), torch.zeros(4),
                                     torch.zeros(1, 1), torch.zeros(1), chunk_size=4, max_seq_len=4, scale=1.0)
    with pytest.raises(ValueError, match="key_cache must have shape"):
        paged_chunk_attention_scores(torch.zeros(1, 4, 32), torch.zeros(1, 32), torch.zeros(4),
                                     torch.zeros(1, 1), torch.zeros(1), chunk_size=4, max_seq_len=4, scale=1.0)
    raw = torch.zeros((2, 8, 1, 32))
    with pytest.raises(ValueError, match="raw key/value must have matching 4-D shapes"):
        rebuild_compact_kv_from_plan(raw, raw[:1], raw, raw, torch.zeros((1, 9), dtype=torch.int64),
                                     torch.zeros((8, 32)), chunk_size=2, max_width=2, rotary_dim=32,
                                     is_neox_style=True)
    with pytest.raises(ValueError, match="working cache slot, head and head dimensions must match raw KV"):
        work = torch.zeros((3, 1, 8, 32))
        rebuild_compact_kv_from_plan(raw, raw, work, work, torch.zeros((1, 9), dtype=torch.int64),
                                     torch.zeros((8, 32)), chunk_size=2, max_width=2, rotary_dim=32,
                                     is_neox_style=True)


def test_step_workspace_size():
    """Header (64 B), a 1 KiB tagged plan copy per row, 4-byte task states
    (ceil(token_budget / 8) per row, rounded up to 256 B), 8-byte tagged partials."""
    from ds355 import _lib

    lib = _lib.load()
    assert lib.ds_step_workspace_bytes(3, 10, 4, 2048) == 64 + 3 * 1024 + 3 * 256 * 4 + 3 * 10 * 4 * 8
    assert lib.ds_step_workspace_bytes(17, 640, 4, 100) == 64 + 17 * 1024 + 1024 + 17 * 640 * 4 * 8  # 17 * 13 * 4 -> 1024
    assert lib.ds_step_workspace_bytes(0, 10, 4, 2048) == 0
    assert lib.ds_step_workspace_bytes(3, 0, 4, 2048) == 0
    assert lib.ds_step_workspace_bytes(3, 10, 4, 0) == 0


def test_attention_workspace_size():
    """256 header bytes, 65536 4-byte span counters, one 8-byte seen word per
    workgroup of the pending rows (rows x Hkv x ceil(G / 16) x spans, rounded
    up to 256 bytes), then fp32 partials: 16 x (D + 4) x 4 bytes per
    workgroup."""
    from ds355 import _lib

    lib = _lib.load()

    def expected(units, d):
        return 256 + 65536 * 4 + (units * 8 + 255) // 256 * 256 + units * 16 * (d + 4) * 4

    assert lib.ds_draft_attention_workspace_bytes(16, 32, 4, 128, 2048) == expected(16 * 4 * 1 * 8, 128)
    # G = 32 -> two query blocks; head_dim 256 -> 128-token spans
    assert lib.ds_draft_attention_workspace_bytes(3, 64, 2, 256, 2048) == expected(3 * 2 * 2 * 16, 256)
    assert lib.ds_draft_attention_workspace_bytes(2, 8, 8, 64, 100) == expected(2 * 8 * 1 * 1, 64)
    assert lib.ds_draft_attention_workspace_bytes(0, 32, 4, 128, 2048) == 0
    assert lib.ds_draft_attention_workspace_bytes(4, 6, 4, 128, 2048) == 0  # 6 query heads over 4 KV heads


def test_attention_validation_without_gpu():
    """The attention entry point checks its arguments before any HIP call."""
    from ds355 import _lib

    lib = _lib.load()

    def call(**kw):
        args = dict(dtype=_lib.DS_BF16, rows=1, out_rows=1, num_slots=1, hq=8, hkv=2, d=128, budget=64,
                    ws=None, ws_bytes=0, ptr=None)
        args.update(kw)
        p = args["ptr"]
        return lib.ds_draft_attention(None, args["dtype"], p, 1024, 128, p, 256, 128, p, 256, 128, p, 1024, 128,
                                      p, p, p, p, None, args["rows"], args["out_rows"], args["num_slots"],
                                      args["hq"], args["hkv"], args["d"], args["budget"], 0.1, args["ws"],
                                      args["ws_bytes"])

    assert call(hq=6, hkv=4) == _lib.DS_ERR_INVALID
    assert "multiple of KV heads" in lib.ds_last_error().decode()
    assert call(rows=2, out_rows=1) == _lib.DS_ERR_INVALID
    assert call(d=96) == _lib.DS_ERR_UNSUPPORTED
    assert call(dtype=_lib.DS_FP32) == _lib.DS_ERR_UNSUPPORTED
    assert call() == _lib.DS_ERR_INVALID  # null pointers
    assert "null tensor pointer" in lib.ds_last_error().decode()
    assert call(rows=0, out_rows=0) == _lib.DS_OK  # nothing to do, nothing launched


def test_attention_refuses_cpu_tensors():
    from ds355.attention import draft_linear_attention

    q = torch.zeros((2, 8, 64), dtype=torch.bfloat16)
    kv = torch.zeros((2, 2, 64), dtype=torch.bfloat16)
    work = torch.zeros((2, 2, 32, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        draft_linear_attention(q, kv, kv, torch.zeros_like(q), work, work.clone(), torch.zeros(2, dtype=torch.int32),
                               [0, 1], [3, 4], scale=0.125, workspace=torch.zeros(16, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="DiffSpec working cache exhausted"):
        draft_linear_attention(q, kv, kv, torch.zeros_like(q), work, work.clone(), torch.zeros(2, dtype=torch.int32),
                               [0, 1], [3, 32], scale=0.125, workspace=torch.zeros(16, dtype=torch.uint8))


def test_capture_validation_without_gpu():
    """The capture entry point checks its arguments before any HIP call."""
    from ds355 import _lib

    lib = _lib.load()

    def call(**kw):
        args = dict(dtype=_lib.DS_BF16, tokens=1, count=1, prev=0, slots=4, lmax=16, heads=2, d=64, wl=None,
                    local=None, rope=None)
        args.update(kw)
        return lib.ds_capture_raw_kv(None, args["dtype"], None, 128, 64, None, 128, 64, None, 0, None,
                                     args["tokens"], None, None, args["slots"], args["lmax"], args["heads"],
                                     args["d"], args["wl"], args["local"], args["rope"], args["count"], args["prev"],
                                     None)

    assert call(tokens=2, count=1) == _lib.DS_ERR_INVALID
    assert "exceed the position count" in lib.ds_last_error().decode()
    assert call(tokens=-1) == _lib.DS_ERR_INVALID
    assert call(dtype=7) == _lib.DS_ERR_INVALID
    assert call(wl=8, local=8) == _lib.DS_ERR_INVALID
    assert "not both" in lib.ds_last_error().decode()
    assert call() == _lib.DS_ERR_INVALID
    assert "null tensor pointer" in lib.ds_last_error().decode()
    assert call(tokens=0, count=0, prev=0) == _lib.DS_OK


def test_capture_refuses_cpu_tensors():
    from ds355.capture import capture_raw_kv_rows

    raw = torch.zeros((2, 8, 1, 64), dtype=torch.bfloat16)
    key = torch.zeros((1, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        capture_raw_kv_rows(key, key, raw, raw.clone(), torch.zeros(1, dtype=torch.int32),
                            torch.zeros(1, dtype=torch.int64), torch.zeros(4, dtype=torch.int64), tokens=1)
    with pytest.raises(RuntimeError, match="exceeds its persistent buffer"):
        capture_raw_kv_rows(key, key, raw, raw.clone(), torch.zeros(1, dtype=torch.int32),
                            torch.zeros(5, dtype=torch.int64), torch.zeros(4, dtype=torch.int64), tokens=1)


def test_static_scratch_step_rejects_what_does_not_fit():
    """ds_retrieval_step_static checks its limits on the host, before any HIP call."""
    from ds355 import _lib

    lib = _lib.load()
    desc = _lib.StepDesc()
    desc.stages = _lib.DS_STAGE_SCORE | _lib.DS_STAGE_SELECT
    desc.batch_rows, desc.batch_size, desc.max_chunks = 64, 64, 4096
    desc.num_kv_heads, desc.num_q_heads = 8, 64  # 64 x 4096 x 8 x 4 B = 8 MiB of partials > 4 MiB
    desc.lse = 1  # a supplied LSE: only the partials count
    assert lib.ds_retrieval_step_static(None, desc, None) == _lib.DS_ERR_INVALID
    assert b"score partials need 8388608 bytes" in lib.ds_last_error()
    desc.max_chunks, desc.lse = 512, None  # partials fit; pairs: 64 x 64 x 512 x 8 B = 16 MiB > 12 MiB
    assert lib.ds_retrieval_step_static(None, desc, None) == _lib.DS_ERR_INVALID
    assert b"(max, sum) pairs" in lib.ds_last_error()
    desc.score_partials = 64  # caller scratch is refused: it lives in the static array
    assert lib.ds_retrieval_step_static(None, desc, None) == _lib.DS_ERR_INVALID
    assert b"takes no score_partials" in lib.ds_last_error()
    desc.score_partials, desc.lse = None, 1
    for stages in (_lib.DS_STAGE_SELECT, _lib.DS_STAGE_SELECT | _lib.DS_STAGE_PLAN,
                   _lib.DS_STAGE_SELECT | _lib.DS_STAGE_PREFIX):
        # A selection without this call's scoring would rank whatever partials an earlier call left.
        desc.stages = stages
        assert lib.ds_retrieval_step_static(None, desc, None) == _lib.DS_ERR_INVALID
        assert b"selects only after scoring in the same call" in lib.ds_last_error()


def test_static_scratch_single_launch_cases_fit_the_fused_region():
    """The static-scratch GPU test's single-launch batches fit DS_STATIC_FUSED_BYTES, so the static entry hands
    the single launch its workspace (csrc/step_static.hip) rather than falling back to the chain."""
    from ds355 import _lib

    lib = _lib.load()
    fused_region = 8 << 20
    for rows, tokens in ((12 + 2, 20000), (9 + 2, 6000)):  # batch rows include the 2 padding rows
        chunks = (tokens + 63) // 64
        need = lib.ds_step_workspace_bytes(rows, chunks, 4, 2048)
        assert 0 < need <= fused_region, (rows, chunks, need)


def test_hip_runtime_lookup_falls_back(monkeypatch):
    """hip_runtime() finds the HIP runtime torch already loaded, by soname or by its mapped path, and returns None
    (callers then use torch's copies and events) when neither finds it; it never loads a second copy."""
    import ctypes
    import os

    from ds355 import _lib

    assert any("libamdhip64.so" in p for p in _lib._loaded_hip_paths())  # torch's runtime is mapped
    monkeypatch.setattr(_lib, "_hip", None)
    monkeypatch.setattr(_lib, "_hip_looked_up", False)
    tried = []
    real_cdll = ctypes.CDLL

    def only_by_path(name, mode=0):
        tried.append(name)
        if not name.startswith("/"):
            raise OSError(f"{name}: not found")  # as with a torch built for another ROCm major
        assert mode & os.RTLD_NOLOAD
        return real_cdll(name, mode=mode)

    monkeypatch.setattr(ctypes, "CDLL", only_by_path)
    assert _lib.hip_runtime() is not None and tried[:2] == ["libamdhip64.so.7", "libamdhip64.so"]
    monkeypatch.setattr(_lib, "_hip", None)
    monkeypatch.setattr(_lib, "_hip_looked_up", False)
    monkeypatch.setattr(ctypes, "CDLL", lambda name, mode=0: (_ for _ in ()).throw(OSError(name)))
    assert _lib.hip_runtime() is None
