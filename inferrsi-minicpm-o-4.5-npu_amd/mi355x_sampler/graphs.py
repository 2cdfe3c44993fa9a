"""HIP-graph decode bodies around the sampling kernel: the Talker post graph and K-frame sample blocks.

* ``TalkerPostGraphs`` is the drop-in for ``engine/runtime/talker_post_graph.py:22-169`` (``NpuTalkerPostGraphs``):
  per padded batch bucket, one captured graph of the codec head projection, the sampling pipeline, the draw and
  the in-place decode-state advance, replayed once per frame of a K block whose counter uniforms are prepared
  outside capture (``begin``).  The pipeline, draw and state advance are one ``mis_sample`` launch with
  ``MIS_UPDATE_STATE``; the head projection stays a torch GEMM, as in the reference.
* ``SampleBlockGraph`` captures K consecutive sample steps of one or more row groups (any vocabulary, dtype and
  semantics) as ONE graph: the K frames' logits are staged in static ``[K, rows, V]`` buffers, their uniforms in
  ``[K, rows]`` buffers filled before each replay, and the history / steps / finished tensors advance inside the
  graph from frame to frame (the sampler half of ``engine/runtime/talker_block_graph.py:92-125``; the model forward
  that produces the logits there is not part of this path).

Captures run on a private stream: the sampler's workspace belongs to the stream a launch is issued on, so every
graph keeps the workspace of its own capture stream (warmed up eagerly on that stream before capture).  Replays of
graphs that share a capture stream must not overlap.
"""

from __future__ import annotations

from contextlib import nullcontext

import torch
import torch.nn.functional as F

from . import talker_sampler as ts
from .groups import RowGroup, launch


def _group(logits, st: dict, cfg: ts.TalkerSampling, eos: int, uniforms, tokens) -> RowGroup:
    return ts._cfg_group(logits, st["history"], st["steps"], eos, cfg, active=st["active"], finished=st["finished"],
                         update_state=True, uniforms=uniforms, tokens=tokens)


class TalkerPostGraphs:
    """``engine/runtime/talker_post_graph.py:22``: one graph per padded batch bucket, replayed once per frame."""

    BUCKETS = (1, 2, 4, 8, 16, 32)

    def __init__(self, head: torch.Tensor, eos: int, cfg: ts.TalkerSampling):
        if head.device.type != "cuda":
            raise ValueError("the codec head must be on the GPU")
        self.head, self.eos, self.cfg = head, int(eos), cfg
        self.device = head.device
        self.pool = torch.cuda.graph_pool_handle()
        self.stream = torch.cuda.Stream(device=self.device)
        self.graphs: dict[int, tuple] = {}
        self.failures: dict[int, str] = {}
        self.replays: dict[int, int] = {}
        self.capture_context = nullcontext
        self._bound: tuple[int, int, ts.DecodeState] | None = None
        self._uniforms: torch.Tensor | None = None
        self._step_index = 0

    def _bucket(self, n: int) -> int:
        for b in self.BUCKETS:
            if b >= n:
                return b
        raise ValueError(f"batch {n} exceeds the largest post-graph bucket {self.BUCKETS[-1]}")

    def _state(self, rows: int) -> dict[str, torch.Tensor]:
        dev = self.device
        z64 = lambda *s: torch.zeros(*s, dtype=torch.int64, device=dev)  # noqa: E731
        zb = lambda *s: torch.zeros(*s, dtype=torch.bool, device=dev)  # noqa: E731
        return {"hidden": self.head.new_zeros((rows, self.head.shape[1])), "seeds": z64(rows),
                "uniform": torch.zeros(rows, dtype=torch.float32, device=dev), "steps": z64(rows),
                "history": torch.full((rows, self.cfg.window), ts.PAD, dtype=torch.int64, device=dev),
                "finished": zb(rows), "active": zb(rows), "out": z64(rows), "feed": z64(rows)}

    def _body(self, st: dict[str, torch.Tensor]) -> None:
        # engine/runtime/talker_post_graph.py:56-76: projection, pipeline + draw with the prepared uniform, and the
        # in-place advance (inside the kernel: live rows only, after every read of the old state)
        logits = F.linear(st["hidden"], self.head).float()
        launch([_group(logits, st, self.cfg, self.eos, st["uniform"], st["out"])])
        st["feed"].copy_(st["out"].clamp_min(0))

    @torch.inference_mode()
    def _capture(self, rows: int) -> tuple:
        with self.capture_context():
            st = self._state(rows)
            snap = {k: v.clone() for k, v in st.items()}
            self.stream.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(self.stream):
                self._body(st)  # eager warm-up on the capture stream: its workspace and the alpha table exist
            torch.cuda.synchronize(self.device)
            for k, v in snap.items():
                st[k].copy_(v)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self.pool, stream=self.stream, capture_error_mode="thread_local"):
                self._body(st)
            torch.cuda.synchronize(self.device)
        self.graphs[rows] = (graph, st)
        return graph, st

    @torch.inference_mode()
    def begin(self, state: ts.DecodeState, *, frames: int = 1) -> bool:
        """``talker_post_graph.py:96-135``: binds ``state`` and prepares the block's uniforms outside capture."""
        if frames < 1:
            raise ValueError("post-graph block must have at least one frame")
        if self.cfg.uses_native_rng:
            raise ValueError("the post graph draws with counter uniforms; native generators are host-driven")
        n = int(state.steps.shape[0])
        rows = self._bucket(n)
        if rows in self.failures:
            return False
        if rows not in self.graphs:
            try:
                self._capture(rows)
            except Exception as exc:  # recorded like the reference; the caller falls back to eager steps
                self.failures[rows] = f"{type(exc).__name__}: {exc}"
                return False
        _, st = self.graphs[rows]
        st["seeds"][:n].copy_(state.seeds)
        st["steps"][:n].copy_(state.steps)
        st["history"][:n].copy_(state.history)
        st["finished"][:n].copy_(state.finished)
        st["active"][:n].copy_(state.active)
        if rows > n:
            st["seeds"][n:].zero_()
            st["steps"][n:].zero_()
            st["history"][n:].fill_(ts.PAD)
            st["finished"][n:].fill_(True)
            st["active"][n:].fill_(False)
            st["uniform"][n:].fill_(0.5)
        offsets = torch.arange(frames, dtype=torch.int64, device=self.device)[:, None]
        self._uniforms = ts.uniform(state.seeds[None, :].expand(frames, n), state.steps[None, :] + offsets)
        self._step_index = 0
        self._bound = (n, rows, state)
        return True

    @torch.inference_mode()
    def step(self, hidden: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """``talker_post_graph.py:137-157``: one replay; returns (tokens, feed = tokens clamped at 0)."""
        if self._bound is None:
            raise RuntimeError("Talker post graph is not bound")
        n, rows, _ = self._bound
        if self._uniforms is None or self._step_index >= self._uniforms.shape[0]:
            raise RuntimeError("post graph exhausted its prepared block uniforms")
        graph, st = self.graphs[rows]
        st["hidden"][:n].copy_(hidden)
        st["uniform"][:n].copy_(self._uniforms[self._step_index])
        self._step_index += 1
        if rows > n:
            st["hidden"][n:].zero_()
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        graph.replay()
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        self.replays[rows] = self.replays.get(rows, 0) + 1
        return st["out"][:n].clone(), st["feed"][:n]

    @torch.inference_mode()
    def finish(self) -> None:
        """``talker_post_graph.py:159-169``: copies the advanced state back into the bound ``DecodeState``."""
        if self._bound is None:
            return
        n, rows, state = self._bound
        _, st = self.graphs[rows]
        state.steps.copy_(st["steps"][:n])
        state.history.copy_(st["history"][:n])
        state.finished.copy_(st["finished"][:n])
        self._bound = None
        self._uniforms = None
        self._step_index = 0


def block_uniforms(seeds: torch.Tensor, steps: torch.Tensor, frames: int, rng: str = "counter",
                   row_ids: torch.Tensor | None = None) -> torch.Tensor:
    """[frames, rows] draws of the next ``frames`` steps, computed outside capture (``talker_block_graph.py:
    92-94``): frame f uses step ``steps + f``."""
    off = torch.arange(frames, dtype=torch.int64, device=seeds.device)[:, None]
    s = seeds.to(torch.int64)[None, :].expand(frames, -1)
    t = steps.to(torch.int64)[None, :] + off
    if rng == "counter":
        return ts.uniform(s, t)
    if rng == "philox":
        rid = torch.zeros_like(seeds, dtype=torch.int64) if row_ids is None else row_ids.to(torch.int64)
        return ts.philox_uniform(s, t, rid[None, :].expand(frames, -1))
    raise ValueError(f"unknown RNG mode: {rng!r}")


class SampleBlockGraph:
    """K sample steps of several row groups as one captured graph, with the decode state advanced in place.

    ``specs``: one dict per group with ``logits`` (a ``[rows, V]`` tensor giving shape and dtype) and the
    ``groups.RowGroup`` keyword arguments of that group (its state tensors — ``history``, ``steps``, ``finished``,
    ``active``, ``history_head`` — are used in place; ``seeds`` / ``uniforms`` / ``tokens`` / ``update_state`` are
    set here).  ``run`` stages the K frames' logits and uniforms, replays, and returns each group's ``[K, rows]``
    tokens.
    """

    def __init__(self, specs: list[dict], frames: int):
        if frames < 1:
            raise ValueError("a block needs at least one frame")
        if not specs:
            raise ValueError("a block needs at least one group")
        self.frames = int(frames)
        self.device = specs[0]["logits"].device
        self.stream = torch.cuda.Stream(device=self.device)
        self.pool = torch.cuda.graph_pool_handle()
        self.logits, self.uniforms, self.tokens, self._frames = [], [], [], []
        for sp in specs:
            x = sp["logits"]
            kw = {k: v for k, v in sp.items() if k != "logits"}
            for k in ("seeds", "uniforms", "tokens", "update_state", "processed", "probs"):
                kw.pop(k, None)
            rows = x.shape[0]
            self.logits.append(torch.zeros((self.frames, *x.shape), dtype=x.dtype, device=self.device))
            self.uniforms.append(torch.full((self.frames, rows), 0.5, dtype=torch.float32, device=self.device))
            self.tokens.append(torch.zeros((self.frames, rows), dtype=torch.int64, device=self.device))
            self._frames.append(kw)
        self.groups = [[RowGroup(self.logits[i][f], **self._frames[i], uniforms=self.uniforms[i][f],
                                 tokens=self.tokens[i][f], update_state=True) for i in range(len(specs))]
                       for f in range(self.frames)]
        self.graph = None

    def _body(self) -> None:
        for grs in self.groups:
            launch(grs)

    def _state_tensors(self) -> list[torch.Tensor]:
        out = []
        for kw in self._frames:
            for k in ("history", "steps", "finished", "history_head"):
                if kw.get(k) is not None:
                    out.append(kw[k])
        return out

    def capture(self) -> None:
        """Warms the capture stream's workspace with one eager pass (the state is restored afterwards), then
        captures the K launches."""
        state = self._state_tensors()
        snap = [t.clone() for t in state]
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            self._body()
        torch.cuda.synchronize(self.device)
        for t, s in zip(state, snap):
            t.copy_(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool, stream=self.stream, capture_error_mode="thread_local"):
            self._body()
        torch.cuda.synchronize(self.device)
        self.graph = graph

    def run(self, logits: list[torch.Tensor], uniforms: list[torch.Tensor]) -> list[torch.Tensor]:
        """One block: ``logits[i]`` is group i's ``[K, rows, V]`` frames, ``uniforms[i]`` its ``[K, rows]`` draws."""
        if len(logits) != len(self.logits) or len(uniforms) != len(self.uniforms):
            raise ValueError("one logits block and one uniform block per group")
        for dst, src in zip(self.logits, logits):
            dst.copy_(src)
        for dst, src in zip(self.uniforms, uniforms):
            dst.copy_(src)
        if self.graph is None:
            self.capture()
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        self.graph.replay()
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        return [t.clone() for t in self.tokens]
