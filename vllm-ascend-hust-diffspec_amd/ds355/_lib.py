"""ctypes binding of libds355.so (the C ABI declared in include/ds355.h).

The library is required: importing a function that needs it on a machine
where it was not built raises, and every entry point checks that its tensors
live on a GPU.  There is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libds355.so"

DS_OK, DS_ERR_INVALID, DS_ERR_UNSUPPORTED, DS_ERR_HIP = 0, 1, 2, 3
DS_BF16, DS_FP16, DS_FP32 = 0, 1, 2
DS_HEAD_MEAN, DS_HEAD_MAX = 0, 1
DS_STAGE_SCORE, DS_STAGE_SELECT, DS_STAGE_PLAN, DS_STAGE_ALL, DS_STAGE_PREFIX = 1, 2, 4, 7, 8
DS_STEP_SELECTORS_GATHER, DS_STEP_EXPIRE_WAITS = 1, 2
# Regions of the static scratch of ds_retrieval_step_static (include/ds355.h).
DS_STATIC_FUSED_BYTES, DS_STATIC_PARTIALS_BYTES, DS_STATIC_PAIRS_BYTES = 8 << 20, 4 << 20, 12 << 20
ABI_VERSION = 7

EXPORTED_SYMBOLS = (
    "ds_last_error",
    "ds_abi_version",
    "ds_chunk_scores",
    "ds_select_chunks",
    "ds_build_plan",
    "ds_rebuild_compact_kv",
    "ds_retrieval_step",
    "ds_retrieval_step_static",
    "ds_step_workspace_bytes",
    "ds_draft_attention",
    "ds_draft_attention_workspace_bytes",
    "ds_capture_raw_kv",
)

_DTYPES = {torch.bfloat16: DS_BF16, torch.float16: DS_FP16, torch.float32: DS_FP32}

# Host-side checks of the preconditions the reference leaves to its callers
# (distinct slots across plan rows, in-range plan entries;
# diffspec/compact_kv.py:199-205).  They read device values back, so they
# are off unless DS355_DEBUG_CHECKS is set to a value other than "" or "0".
DEBUG_CHECKS = os.environ.get("DS355_DEBUG_CHECKS", "0") not in ("", "0")

_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class UnsupportedShapeError(ValueError):
    """A valid request outside what the HIP kernels cover."""


class StepDesc(ctypes.Structure):
    """Mirror of ``ds_step_desc`` (include/ds355.h)."""

    _fields_ = [
        ("dtype", _i32),
        ("query", _p), ("q_stride", _i64),
        ("lse", _p), ("lse_token_stride", _i64), ("lse_head_stride", _i64),
        ("key_cache", _p), ("k_block_stride", _i64), ("k_token_stride", _i64), ("k_head_stride", _i64),
        ("block_size", _i32),
        ("block_table", _p), ("bt_stride", _i64),
        ("counts", _p), ("query_start", _p), ("query_len", _p), ("target_len", _p),
        ("batch_rows", _i32), ("batch_size", _i32),
        ("num_q_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("scale", _f32),
        ("max_chunks", _i32),
        ("scores", _p),
        ("score_partials", _p),
        ("stages", _i32),
        ("sel_ids", _p), ("sel_stride", _i64), ("sel_count", _p), ("slots", _p),
        ("committed_lens", _p), ("plan", _p), ("plan_width", _i32), ("working_lens", _p),
        ("kv_dtype", _i32),
        ("raw_key", _p), ("raw_value", _p), ("working_key", _p), ("working_value", _p),
        ("num_slots", _i32), ("max_model_len", _i32), ("draft_heads", _i32), ("draft_head_dim", _i32),
        ("token_budget", _i32),
        ("cos_sin", _p), ("cs_stride", _i64), ("cs_rows", _i32),
        ("rotary_dim", _i32), ("is_neox_style", _i32),
        ("row_active", _p),
        ("chunk_size", _i32), ("history_budget", _i32), ("recent_window", _i32),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
        ("lse_partials", _p), ("lse_out", _p), ("lse_out_stride", _i64),
        ("flags", _i32),
        ("sel_gen", _p), ("gather_rec", _p), ("rec_stride", _i64),
    ]


_SIGNATURES = {
    "ds_last_error": (ctypes.c_char_p, []),
    "ds_abi_version": (_i32, []),
    "ds_chunk_scores": (_i32, [
        _p, _i32, _p, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _p,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _p, _i64, _p, ctypes.c_size_t,
    ]),
    "ds_select_chunks": (_i32, [_p, _p, _i64, _i32, _p, _i32, _i32, _i32, _p, _i64, _p]),
    "ds_build_plan": (_i32, [_p, _p, _i64, _p, _i32, _p, _p, _i32, _i32, _i32, _i32, _p, _i32, _p]),
    "ds_rebuild_compact_kv": (_i32, [
        _p, _i32, _p, _p, _p, _p, _p, _i32, _i32, _p, _i64, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p,
    ]),
    "ds_retrieval_step": (_i32, [_p, ctypes.POINTER(StepDesc)]),
    "ds_retrieval_step_static": (_i32, [_p, ctypes.POINTER(StepDesc), _p]),
    "ds_step_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32, _i32]),
    "ds_draft_attention": (_i32, [
        _p, _i32, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64,
        _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p, ctypes.c_size_t,
    ]),
    "ds_draft_attention_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32, _i32, _i32]),
    "ds_capture_raw_kv": (_i32, [
        _p, _i32, _p, _i64, _i64, _p, _i64, _i64, _p, _i32, _p, _i32, _p, _p,
        _i32, _i32, _i32, _i32, _p, _p, _p, _i32, _i32, _p,
    ]),
}

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library once; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"{LIBRARY_PATH} is missing: build it with `python -m ds355.build` "
            "(hipcc, gfx950). ds355 has no CPU fallback."
        )
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.ds_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libds355 ABI version {version} != expected {ABI_VERSION}: rebuild the library")
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc == DS_OK:
        return
    message = load().ds_last_error().decode(errors="replace")
    if rc == DS_ERR_INVALID:
        raise ValueError(message)
    if rc == DS_ERR_UNSUPPORTED:
        raise UnsupportedShapeError(message)
    raise RuntimeError(f"libds355: {message}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# torch's own getter of the current stream's raw handle (what its compiled
# kernels launch on); a few microseconds cheaper than building a Stream object.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)

_hip: ctypes.CDLL | None = None
_hip_looked_up = False
HIP_MEMCPY_HOST_TO_DEVICE = 1
HIP_EVENT_DISABLE_TIMING = 2


def _loaded_hip_paths() -> list[str]:
    """Paths of HIP runtimes already mapped into this process (torch's), by /proc/self/maps."""
    paths: list[str] = []
    try:
        with open("/proc/self/maps") as maps:
            for line in maps:
                path = line.rstrip("\n").split(maxsplit=5)[-1]
                if "/libamdhip64.so" in path and path not in paths:
                    paths.append(path)
    except OSError:
        pass
    return paths


def hip_runtime() -> ctypes.CDLL | None:
    """The HIP runtime already loaded in the process (torch's, which the
    library's kernels and streams share), for small host-side copies and
    events without torch's dispatch cost.  Never loads a second copy: it is
    looked up by soname, then by the path mapped into the process, with
    RTLD_NOLOAD.  None when neither finds it; callers then use torch's
    copies and events."""
    global _hip, _hip_looked_up
    if _hip_looked_up:
        return _hip
    _hip_looked_up = True
    hip = None
    for name in ("libamdhip64.so.7", "libamdhip64.so", *_loaded_hip_paths()):
        try:
            hip = ctypes.CDLL(name, mode=os.RTLD_NOLOAD | os.RTLD_LAZY)
            break
        except OSError:
            continue
    if hip is None:
        return None
    hip.hipMemcpyAsync.restype = ctypes.c_int
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    hip.hipEventCreateWithFlags.restype = ctypes.c_int
    hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
    hip.hipEventRecord.restype = ctypes.c_int
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventSynchronize.restype = ctypes.c_int
    hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipEventDestroy.restype = ctypes.c_int
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    _hip = hip
    return _hip


def hip_check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with HIP error {rc}")


def stream_handle(device: torch.device) -> int:
    """Raw HIP handle of torch's current stream on ``device``."""
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    """All tensors on one GPU; ds355 has no CPU path."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"ds355 runs on the GPU only; got a tensor on {t.device}")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("KV caches, plan and cos/sin cache must share a device")
    if device is None:
        raise ValueError("no tensor given")
    return device
