"""Row groups: the per-row sampling API on device tensors, one fused launch for any number of groups.

A ``RowGroup`` is every row of one logits matrix (one vocabulary size, dtype
and pipeline order) with its per-row parameters and decode state; ``launch``
samples several groups (e.g. Thinker rows at V = 151,748 bf16 and Talker rows
at V = 6,562 fp32) in a single kernel launch.  Nothing here reads device data
on the host or synchronises, so a launch can be captured into a graph.

Row semantics are the reference pipeline (``engine/talker_sampler.py:136-172``)
generalised to per-row parameters, with vLLM's sentinels when
``top_k_zero_disables`` / ``top_p_one_disables`` are set (the defaults here):
``top_k <= 0`` keeps the whole vocabulary, ``top_p >= 1`` skips top-p, and
``temperature <= 0`` selects greedily.
"""

from __future__ import annotations

import torch

from . import _lib

_SEMANTICS = {"omni": _lib.MIS_OMNI, "hf": _lib.MIS_HF}
_RNG = {"counter": _lib.MIS_RNG_COUNTER, "philox": _lib.MIS_RNG_PHILOX}


def _require_device(t: torch.Tensor, name: str, device: torch.device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU (the sampler has no CPU path); got {t.device}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, logits on {device}")


class RowGroup:
    """One group of rows; see ``include/mi355x_sampler.h`` for the field meanings.

    Per-row parameters take a Python number (every row) or a ``[rows]`` device tensor.  Output arguments take
    ``True`` (allocate), ``False`` / ``None`` (skip) or a device tensor to write into.
    """

    def __init__(self, logits: torch.Tensor, *, temperature=1.0, top_k=0, top_p=1.0, repetition=1.0, presence=0.0,
                 frequency=0.0, history: torch.Tensor | None = None, history_head: torch.Tensor | None = None,
                 allowed: torch.Tensor | None = None, eos: int = -1, min_new_tokens: int = 0, max_new_tokens: int = 0,
                 seeds: torch.Tensor | None = None, steps: torch.Tensor | None = None,
                 row_ids: torch.Tensor | None = None, uniforms: torch.Tensor | None = None,
                 active: torch.Tensor | None = None, finished: torch.Tensor | None = None, semantics: str = "omni",
                 min_keep: int = 1, rng: str = "counter", top_k_zero_disables: bool = True,
                 top_p_one_disables: bool = True, update_state: bool = False, tokens=True, processed=False,
                 probs=False, alpha_lut: torch.Tensor | None = None, finalize_streaming: bool = False):
        if not isinstance(logits, torch.Tensor) or logits.dim() != 2:
            raise ValueError("logits must be a [rows, vocab] tensor")
        self.device = logits.device
        _require_device(logits, "logits", self.device)
        if logits.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"logits dtype must be float32 or bfloat16, got {logits.dtype}")
        if logits.stride(-1) != 1:
            logits = logits.contiguous()
        if semantics not in _SEMANTICS:
            raise ValueError(f"unknown Talker sampling semantics: {semantics!r}")
        if rng not in _RNG:
            raise ValueError(f"unknown RNG mode: {rng!r}")
        self.rows, self.vocab = int(logits.shape[0]), int(logits.shape[1])
        self._keep: list[torch.Tensor] = [logits]
        g = _lib.MisGroup()
        g.logits = logits.data_ptr()
        g.logits_row_stride = logits.stride(0) if self.rows > 1 else self.vocab
        g.dtype = _lib.MIS_BF16 if logits.dtype == torch.bfloat16 else _lib.MIS_F32
        g.vocab, g.rows = self.vocab, self.rows
        g.semantics = _SEMANTICS[semantics]
        g.min_keep = int(min_keep)
        g.flags = ((_lib.MIS_TOPK_ZERO_DISABLES if top_k_zero_disables else 0)
                   | (_lib.MIS_TOPP_ONE_DISABLES if top_p_one_disables else 0)
                   | (_lib.MIS_UPDATE_STATE if update_state else 0)
                   | (_lib.MIS_FINALIZE_STREAMING if finalize_streaming else 0))
        g.temperature, g.temperature_value = self._param(temperature, torch.float32, "temperature")
        g.top_k, g.top_k_value = self._param(top_k, torch.int32, "top_k")
        g.top_p, g.top_p_value = self._param(top_p, torch.float32, "top_p")
        g.repetition, g.repetition_value = self._param(repetition, torch.float32, "repetition")
        g.presence, g.presence_value = self._param(presence, torch.float32, "presence")
        g.frequency, g.frequency_value = self._param(frequency, torch.float32, "frequency")
        if alpha_lut is not None:
            lut = self._vec(alpha_lut, torch.float32, "alpha_lut", None)
            g.alpha_lut, g.alpha_lut_len = lut.data_ptr(), lut.numel()
        if history is not None:
            _require_device(history, "history", self.device)
            if history.dim() != 2 or history.shape[0] != self.rows:
                raise ValueError("history must be [rows, window]")
            if history.dtype not in (torch.int32, torch.int64):
                raise ValueError("history must be int32 or int64")
            if history.shape[1] > 0 and history.stride(-1) != 1:
                raise ValueError("history rows must be contiguous (it is updated in place)")
            self._keep.append(history)
            g.history = history.data_ptr()
            g.history_len = int(history.shape[1])
            g.history_row_stride = history.stride(0) if self.rows > 1 else max(1, g.history_len)
            g.history_is_int64 = int(history.dtype == torch.int64)
            g.history_mode = _lib.MIS_HISTORY_WINDOW
            if history_head is not None:
                head = self._state(history_head, torch.int32, "history_head")
                g.history_mode = _lib.MIS_HISTORY_RING
                g.history_head = head.data_ptr()
        if allowed is not None:
            _require_device(allowed, "allowed", self.device)
            if allowed.dtype != torch.int32 or allowed.dim() != 2 or allowed.shape[0] != self.rows:
                raise ValueError("allowed must be a [rows, ceil(vocab/32)] int32 bitmask")
            if allowed.shape[1] < (self.vocab + 31) // 32 or allowed.stride(-1) != 1:
                raise ValueError("allowed must hold ceil(vocab/32) contiguous words per row")
            self._keep.append(allowed)
            g.allowed = allowed.data_ptr()
            g.allowed_row_stride = allowed.stride(0) if self.rows > 1 else allowed.shape[1]
        g.eos, g.min_new_tokens, g.max_new_tokens = int(eos), int(min_new_tokens), int(max_new_tokens)
        g.rng = _RNG[rng]
        g.seeds = self._vec(seeds, torch.int64, "seeds", self.rows, ptr=True)
        g.steps = self._state(steps, torch.int64, "steps", ptr=True)
        g.row_ids = self._vec(row_ids, torch.int64, "row_ids", self.rows, ptr=True)
        g.uniforms = self._vec(uniforms, torch.float32, "uniforms", self.rows, ptr=True)
        g.active = self._state(active, torch.bool, "active", ptr=True)
        g.finished = self._state(finished, torch.bool, "finished", ptr=True)
        self.tokens = self._out(tokens, (self.rows,), torch.int64, "tokens")
        self.processed = self._out(processed, (self.rows, self.vocab), torch.float32, "processed")
        self.probs = self._out(probs, (self.rows, self.vocab), torch.float32, "probs")
        g.tokens = _lib.ptr(self.tokens)
        g.processed = _lib.ptr(self.processed)
        g.processed_row_stride = self.processed.stride(0) if self.processed is not None and self.rows > 1 else self.vocab
        g.probs = _lib.ptr(self.probs)
        g.probs_row_stride = self.probs.stride(0) if self.probs is not None and self.rows > 1 else self.vocab
        self.struct = g

    # -- helpers
    def _param(self, v, dtype, name):
        if isinstance(v, torch.Tensor):
            t = self._vec(v, dtype, name, self.rows)
            return t.data_ptr(), 0
        return None, (float(v) if dtype == torch.float32 else int(v))

    def _vec(self, v, dtype, name, n, ptr=False):
        if v is None:
            return None
        _require_device(v, name, self.device)
        if n is not None and v.numel() != n:
            raise ValueError(f"{name} must have {n} entries, got {v.numel()}")
        t = v.reshape(-1)
        if t.dtype != dtype or not t.is_contiguous():
            t = t.to(dtype).contiguous()
        self._keep.append(t)
        return t.data_ptr() if ptr else t

    def _state(self, v, dtype, name, ptr=False):
        """Decode state that the kernel may update in place: must already have the right dtype and layout."""
        if v is None:
            return None
        _require_device(v, name, self.device)
        if v.dtype != dtype or not v.is_contiguous() or v.numel() != self.rows:
            raise ValueError(f"{name} must be a contiguous [{self.rows}] {dtype} tensor")
        self._keep.append(v)
        return v.data_ptr() if ptr else v

    def _out(self, spec, shape, dtype, name):
        if spec is None or spec is False:
            return None
        if spec is True:
            return torch.empty(shape, dtype=dtype, device=self.device)
        _require_device(spec, name, self.device)
        if spec.dtype != dtype or tuple(spec.shape) != tuple(shape) or spec.stride(-1) != 1:
            raise ValueError(f"{name} must be a {tuple(shape)} {dtype} tensor with contiguous rows")
        return spec


def launch(groups: list[RowGroup]) -> None:
    """Samples every group in one kernel launch on the current stream of their device."""
    if not groups:
        return
    dev = groups[0].device
    for g in groups[1:]:
        if g.device != dev:
            raise ValueError("all groups of a launch must be on one device")
    _lib.sample([g.struct for g in groups], dev)


def launch_static(groups: list[RowGroup]) -> None:
    """``launch`` on the library's own workspace (no allocation; launches that overlap on one GPU race)."""
    if not groups:
        return
    dev = groups[0].device
    for g in groups[1:]:
        if g.device != dev:
            raise ValueError("all groups of a launch must be on one device")
    _lib.sample_static([g.struct for g in groups], dev)


def sample(logits: torch.Tensor, **kw) -> RowGroup:
    """One group, one launch; returns the group (``.tokens``, ``.processed``, ``.probs``)."""
    g = RowGroup(logits, **kw)
    launch([g])
    return g


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """Thinker greedy decode: first index of the row maximum (``engine/runtime/thinker_decode.py:107``)."""
    return sample(logits, temperature=0.0).tokens
