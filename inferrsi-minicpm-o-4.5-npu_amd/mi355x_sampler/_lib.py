"""ctypes binding of ``libmi355x_sampler.so`` (the C-ABI declared in ``include/mi355x_sampler.h``).

There is no CPU fallback: every entry point needs the HIP library and device
tensors, and raises when either is missing.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmi355x_sampler.so"

MIS_ABI_VERSION = 1
MIS_F32, MIS_BF16 = 0, 1
MIS_OMNI, MIS_HF = 0, 1
MIS_RNG_COUNTER, MIS_RNG_PHILOX = 0, 1
MIS_HISTORY_WINDOW, MIS_HISTORY_RING = 0, 1
MIS_TOPK_ZERO_DISABLES, MIS_TOPP_ONE_DISABLES, MIS_UPDATE_STATE, MIS_FINALIZE_STREAMING = 1, 2, 4, 8
MIS_E_ARG, MIS_E_WORKSPACE, MIS_E_UNSUPPORTED = 1, 2, 3
MIS_WS_PATH_OFFSET = 64
MIS_WS_ERROR_OFFSET = 128  # u32: slices that gave up waiting for their row's finaliser (include/mi355x_sampler.h)
MIS_STATIC_WORKSPACE_BYTES = 64 << 20
PATHS = ("greedy", "full", "candidates", "histogram", "stream", "forced")  # MIS_PATH_* order

_vp = ctypes.c_void_p
_i32, _i64, _f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float


class MisGroup(ctypes.Structure):
    """Mirror of ``MisGroup`` in ``include/mi355x_sampler.h`` (field order and types must match)."""

    _fields_ = [
        ("logits", _vp), ("logits_row_stride", _i64), ("dtype", _i32), ("vocab", _i32), ("rows", _i32),
        ("semantics", _i32), ("flags", _i32), ("min_keep", _i32),
        ("temperature", _vp), ("top_k", _vp), ("top_p", _vp), ("repetition", _vp), ("presence", _vp),
        ("frequency", _vp),
        ("temperature_value", _f32), ("top_p_value", _f32), ("repetition_value", _f32), ("presence_value", _f32),
        ("frequency_value", _f32), ("top_k_value", _i32),
        ("alpha_lut", _vp), ("alpha_lut_len", _i32), ("history_len", _i32),
        ("history", _vp), ("history_row_stride", _i64), ("history_is_int64", _i32), ("history_mode", _i32),
        ("history_head", _vp),
        ("allowed", _vp), ("allowed_row_stride", _i64),
        ("eos", _i32), ("min_new_tokens", _i32), ("max_new_tokens", _i32), ("rng", _i32),
        ("seeds", _vp), ("steps", _vp), ("row_ids", _vp), ("uniforms", _vp), ("active", _vp), ("finished", _vp),
        ("tokens", _vp), ("processed", _vp), ("processed_row_stride", _i64), ("probs", _vp),
        ("probs_row_stride", _i64),
    ]


EXPORTS = ("mis_version", "mis_sizeof_group", "mis_last_error", "mis_workspace_bytes", "mis_sample", "mis_sample_static",
           "mis_uniform")

_lock = threading.Lock()
_handle: ctypes.CDLL | None = None


class SamplerError(RuntimeError):
    pass


def load(path: Path | str = LIB_PATH) -> ctypes.CDLL:
    """Open the library and declare its signatures (no GPU needed)."""
    if not Path(path).exists():
        raise RuntimeError(f"{path} is missing: build it with inferrsi-minicpm-o-4.5-npu_amd/mi355x_sampler/build.py")
    h = ctypes.CDLL(str(path))
    h.mis_version.restype = ctypes.c_int
    h.mis_sizeof_group.restype = ctypes.c_size_t
    h.mis_last_error.restype = ctypes.c_char_p
    h.mis_workspace_bytes.restype = ctypes.c_size_t
    h.mis_workspace_bytes.argtypes = [ctypes.POINTER(MisGroup), ctypes.c_int]
    h.mis_sample.restype = ctypes.c_int
    h.mis_sample.argtypes = [ctypes.POINTER(MisGroup), ctypes.c_int, _vp, ctypes.c_size_t, _vp]
    h.mis_sample_static.restype = ctypes.c_int
    h.mis_sample_static.argtypes = [ctypes.POINTER(MisGroup), ctypes.c_int, _vp]
    h.mis_uniform.restype = ctypes.c_int
    h.mis_uniform.argtypes = [_vp, _vp, _vp, _i64, _i32, _vp, _vp]
    if h.mis_version() != MIS_ABI_VERSION:
        raise RuntimeError(f"library ABI {h.mis_version()} != binding ABI {MIS_ABI_VERSION}")
    if h.mis_sizeof_group() != ctypes.sizeof(MisGroup):
        raise RuntimeError(f"MisGroup layout mismatch: library {h.mis_sizeof_group()} B, binding {ctypes.sizeof(MisGroup)} B")
    return h


def lib() -> ctypes.CDLL:
    global _handle
    with _lock:
        if _handle is None:
            _handle = load()
        return _handle


def check(rc: int) -> None:
    if rc == 0:
        return
    msg = lib().mis_last_error().decode(errors="replace")
    if rc == MIS_E_ARG or rc == MIS_E_UNSUPPORTED:
        raise ValueError(msg)
    raise SamplerError(f"mi355x sampler failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# Workspace per (device, stream): launches sharing one must be stream-ordered.  A buffer that is outgrown is kept
# alive for the life of the process: a graph captured while it was current still writes to it on every replay.
_ws: dict[tuple[int, int], torch.Tensor] = {}
_retired: list[torch.Tensor] = []


def _ws_key(device: torch.device) -> tuple[int, int]:
    return (device.index if device.index is not None else torch.cuda.current_device(), stream_handle(device))


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    key = _ws_key(device)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _retired.append(buf)
        buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)  # counters start at zero
        _ws[key] = buf
    return buf


def _path_words(device: torch.device) -> torch.Tensor | None:
    buf = _ws.get(_ws_key(device))
    if buf is None:
        return None
    return buf[MIS_WS_PATH_OFFSET:MIS_WS_PATH_OFFSET + 4 * len(PATHS)].view(torch.int32)


def path_counters(device: torch.device) -> dict[str, int]:
    """Rows finalised per path on the workspace of ``device``'s current stream since the last reset (diagnostics;
    reads device memory, so it synchronises)."""
    words = _path_words(device)
    if words is None:
        return dict.fromkeys(PATHS, 0)
    v = words.cpu().tolist()
    return {p: int(v[i]) for i, p in enumerate(PATHS)}


def wait_failures(device: torch.device) -> int:
    """Slices that gave up waiting for their row's finaliser on the workspace of ``device``'s current stream since
    the last reset (0 unless the device stalled a workgroup for milliseconds; synchronises)."""
    buf = _ws.get(_ws_key(device))
    if buf is None:
        return 0
    return int(buf[MIS_WS_ERROR_OFFSET:MIS_WS_ERROR_OFFSET + 4].view(torch.int32).item())


def reset_path_counters(device: torch.device) -> None:
    """Zeroes the path counters and the wait-failure count."""
    words = _path_words(device)
    if words is not None:
        words.zero_()
        _ws[_ws_key(device)][MIS_WS_ERROR_OFFSET:MIS_WS_ERROR_OFFSET + 4].zero_()


def sample(groups: list[MisGroup], device: torch.device) -> None:
    arr = (MisGroup * len(groups))(*groups)
    need = lib().mis_workspace_bytes(arr, len(groups))
    if need == 0 and any(g.rows for g in groups):
        check(lib().mis_sample(arr, len(groups), None, 0, None))  # reports the argument error
    ws = workspace(device, need)
    check(lib().mis_sample(arr, len(groups), ws.data_ptr(), ws.numel(), stream_handle(device)))


def sample_static(groups: list[MisGroup], device: torch.device) -> None:
    """One launch on the library's own workspace (``mis_sample_static``): allocates nothing, for callers that
    cannot allocate; launches that overlap on one GPU race."""
    arr = (MisGroup * len(groups))(*groups)
    check(lib().mis_sample_static(arr, len(groups), stream_handle(device)))


def uniform(seeds: torch.Tensor, steps: torch.Tensor, row_ids: torch.Tensor | None, rng: int) -> torch.Tensor:
    out = torch.empty(seeds.shape, dtype=torch.float32, device=seeds.device)
    check(lib().mis_uniform(ptr(seeds), ptr(steps), ptr(row_ids), seeds.numel(), rng, out.data_ptr(),
                            stream_handle(seeds.device)))
    return out
