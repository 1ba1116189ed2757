"""Decode-step and flow-step HIP graphs.

``DecodeGraphRunner``: one captured graph per KV length, replayed.
``FlowStepGraph`` / ``fuse_flow_graph``: one graph for the fixed-shape flow
ODE step (see their docstrings).

Same contract as the reference's decode runner (src/umic/graph.py:36-176):
the runner wraps the VLM's ``forward`` (instance attribute, so module hooks
still fire) and, during ``generate()``, serves every single-token decode step
from a graph captured once per KV length.  The graphs persist across
inferences: the KV buffers, static inputs and M-RoPE delta live in the
runner, and each new inference copies its prefill KV into them, so captured
graphs keep valid buffer addresses and later inferences are pure replay.
Exact-length graphs keep ``attention_mask=None``, which lets attention use
its fused kernels with grouped-query heads.

On this runtime the cache is ``umic.cache.InplaceKVCache`` in graph mode:
the write position is a device tensor updated before each replay.  With
``umic.integrate.fuse_kv_rope`` applied, every layer's RoPE and KV write
inside the graph is one ``umic_rope_kv_append_bf16`` launch reading that
position (the reference replays RoPE plus two ``index_copy_`` per layer).

Positions.  The installed forward keeps the model's signature, because
``generate()`` picks the inputs it passes by that signature (transformers 5.x
passes ``position_ids`` -- [4, B, 1] text + M-RoPE rows -- and no
``cache_position``).  Each step copies the given position ids into a static
device buffer that the graph reads; the KV write position is the cache length
the runner tracks on the host (no device sync).  Without given position ids
the graph computes them as position + the model's ``rope_deltas`` (the
reference's rule, src/umic/graph.py:128-136).
"""

from __future__ import annotations

import functools
import logging
from typing import Any

import torch
from transformers.cache_utils import DynamicCache

from umic.cache import InplaceKVCache

logger = logging.getLogger(__name__)

# forward() arguments that carry a new multimodal input or replace input_ids:
# such a call is not a plain decode step
_NOT_DECODE = ("inputs_embeds", "pixel_values", "pixel_values_videos")
# arguments the static call supplies itself
_STATIC = ("input_ids", "attention_mask", "past_key_values", "position_ids", "cache_position")


class DecodeGraphRunner:
    """Wraps a VLM's forward; replays per-KV-length graphs for decode."""

    def __init__(self, vlm: torch.nn.Module, max_new_tokens: int = 96,
                 warmup_steps: int = 2) -> None:
        self.vlm = vlm
        self.orig_forward = vlm.forward
        self.max_new = max_new_tokens
        self.warmup_steps = warmup_steps
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.outs: dict[int, Any] = {}
        self.pool = None
        self.cache: InplaceKVCache | None = None   # persistent KV buffers
        self.base_len: int | None = None
        self.in_decode = False
        self.disabled = False
        self.step = 0
        self.replays = 0
        self.s_ids = self.s_pos = self.s_rope = self.s_pids = None
        self.static_kwargs: dict[str, Any] = {}

        @functools.wraps(self.orig_forward)
        def forward(*args: Any, **kwargs: Any):
            return self(*args, **kwargs)

        forward._umic_runner = self
        vlm.forward = forward
        orig_generate = getattr(vlm, "generate", None)
        if orig_generate is not None:
            def _generate(*args: Any, **kwargs: Any):
                try:
                    return orig_generate(*args, **kwargs)
                finally:
                    self.finish()

            vlm.generate = _generate
        logger.info("DecodeGraphRunner installed on %s", type(vlm).__name__)

    # -- inference boundaries ----------------------------------------------

    def finish(self) -> None:
        """generate() returned: leave the cache in dynamic mode."""
        if self.cache is not None:
            self.cache.disable_graph_mode()
        self.in_decode = False
        self.step = 0

    def _is_decode_call(self, args, kwargs) -> bool:
        ids = kwargs.get("input_ids")
        pkv = kwargs.get("past_key_values")
        return (not args and not self.disabled and isinstance(ids, torch.Tensor)
                and ids.is_cuda and tuple(ids.shape) == (1, 1)
                and isinstance(pkv, DynamicCache) and pkv.get_seq_length() > 0
                and all(kwargs.get(k) is None for k in _NOT_DECODE)
                and not torch.cuda.is_current_stream_capturing())

    def _begin_inference(self, kwargs: dict[str, Any]) -> bool:
        """First decode step of a generate() call: bind the persistent cache."""
        pkv = kwargs["past_key_values"]
        if not all(getattr(lyr, "keys", None) is not None for lyr in pkv.layers):
            return False
        mask = kwargs.get("attention_mask")
        if mask is not None and not bool((mask == 1).all().item()):
            logger.warning("DecodeGraphRunner: padded attention mask -- eager decode")
            return False
        base = pkv.get_seq_length()
        if pkv is self.cache:
            pass                                   # continuing on our own buffers
        elif self.cache is not None and base == self.base_len:
            # same prompt length: copy the new prefill KV into the persistent
            # buffers, so the captured graphs' addresses stay valid
            for dst, src in zip(self.cache.layers, pkv.layers):
                dst._k_buf[:, :, :base].copy_(src.keys)
                dst._v_buf[:, :, :base].copy_(src.values)
            self.cache.set_pos(base)
        else:
            if self.cache is not None:
                logger.info("DecodeGraphRunner: prompt length %s -> %d, recapturing",
                            self.base_len, base)
                self.graphs.clear()
                self.outs.clear()
                self.pool = None
            self.cache = InplaceKVCache.from_dynamic(pkv, extra_tokens=self.max_new)
            self.base_len = base
        dev = kwargs["input_ids"].device
        if self.s_ids is None:
            self.s_ids = torch.zeros(1, 1, dtype=torch.long, device=dev)
            self.s_pos = torch.zeros(1, dtype=torch.long, device=dev)
            self.s_rope = torch.zeros(1, dtype=torch.long, device=dev)
        deltas = getattr(getattr(self.vlm, "model", None), "rope_deltas", None)
        if isinstance(deltas, torch.Tensor):
            self.s_rope.copy_(deltas.reshape(-1)[:1])
        else:
            self.s_rope.zero_()
        pids = kwargs.get("position_ids")
        shape = None if pids is None else tuple(pids.shape)
        if (self.s_pids is None) != (pids is None) or (
                pids is not None and tuple(self.s_pids.shape) != shape):
            # the static position input changes form: graphs must be recaptured
            self.graphs.clear()
            self.outs.clear()
            self.s_pids = None if pids is None else torch.zeros(shape, dtype=pids.dtype,
                                                                device=dev)
        self.cache.enable_graph_mode(self.s_pos)
        self.static_kwargs = {k: v for k, v in kwargs.items() if k not in _STATIC}
        self.in_decode = True
        return True

    # -- the captured step ---------------------------------------------------

    def _static_call(self):
        pos = self.s_pids
        if pos is None:
            pos = (self.s_pos + self.s_rope).view(1, 1, 1).expand(3, 1, 1)
        return self.orig_forward(input_ids=self.s_ids, attention_mask=None,
                                 past_key_values=self.cache, position_ids=pos,
                                 **self.static_kwargs)

    def _eager(self, args, kwargs):
        """Run the step eagerly.  A step on the runner's cache leaves graph
        mode first, so it appends at the host-side position."""
        if self.in_decode and kwargs.get("past_key_values") is self.cache:
            self.finish()
        return self.orig_forward(*args, **kwargs)

    def __call__(self, *args: Any, **kwargs: Any):
        if not self._is_decode_call(args, kwargs):
            return self._eager(args, kwargs)
        pkv = kwargs["past_key_values"]
        if (not self.in_decode or pkv is not self.cache) and not self._begin_inference(kwargs):
            return self._eager(args, kwargs)
        pos = self.cache.get_seq_length()           # tokens already cached (host)
        if pos + 1 > self.cache.layers[0].capacity:
            raise RuntimeError(f"DecodeGraphRunner: decode step {pos + 1 - self.base_len} "
                               f"exceeds the cache headroom (max_new_tokens={self.max_new})")
        kv_len = pos + 1
        pids = kwargs.get("position_ids")
        if (pids is None) != (self.s_pids is None) or (
                pids is not None and pids.shape != self.s_pids.shape):
            return self._eager(args, kwargs)             # not the captured form
        self.s_ids.copy_(kwargs["input_ids"])
        self.s_pos.fill_(pos)
        if pids is not None:
            self.s_pids.copy_(pids)
        self.cache.set_graph_len(kv_len)
        if not self.graphs and self.step < self.warmup_steps:
            # lazy library initialisation runs before the first capture
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                out = self._static_call()
            torch.cuda.current_stream().wait_stream(side)
        elif kv_len not in self.graphs:
            try:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=self.pool):
                    self.outs[kv_len] = self._static_call()
            except Exception as exc:  # noqa: BLE001 -- correctness first
                logger.warning("DecodeGraphRunner: capture failed (%s); eager decode", exc)
                self.disabled = True
                self.cache.set_pos(pos)
                return self._eager(args, kwargs)
            if self.pool is None:
                self.pool = graph.pool()
            self.graphs[kv_len] = graph
            graph.replay()
            self.replays += 1
            out = self.outs[kv_len]
        else:
            self.graphs[kv_len].replay()
            self.replays += 1
            out = self.outs[kv_len]
        self.step += 1
        self.cache.set_pos(kv_len)
        return out


def fuse_decode_graph(vlm: torch.nn.Module, max_new_tokens: int = 96) -> DecodeGraphRunner:
    """Install the per-length decode graph runner on the VLM
    (src/umic/graph.py:179-181).  Idempotent: a VLM that already carries a
    runner keeps it (a second one would wrap the first and keep a second KV
    cache)."""
    existing = getattr(getattr(vlm, "forward", None), "_umic_runner", None)
    if isinstance(existing, DecodeGraphRunner):
        existing.max_new = max(existing.max_new, max_new_tokens)
        return existing
    return DecodeGraphRunner(vlm, max_new_tokens=max_new_tokens)


class FlowStepGraph:
    """One captured graph for a fixed-shape flow ODE step, replayed per step.

    Same contract as src/umic/graph.py:179-232.  Every step of the flow
    expert runs ``step_fn(x=, t=)`` on the same shapes: its action tokens are
    appended to the prefix KV at the same cache rows and cropped back, so the
    buffers the kernels touch are identical each step and only the values of
    x and t change.  After ``warmup`` eager steps the step is captured once
    (on static copies of x and t); later steps copy x and t in and replay.
    With ``umic.integrate.fuse_kv_rope`` the attention's RoPE and cache write
    inside the graph is one launch at the baked cache position.  A capture
    that fails falls back to eager for good, so results never depend on it.
    The graph holds the buffer addresses of the cache it was captured on:
    build a new one per inference (per prompt cache).
    """

    def __init__(self, step_fn, warmup: int = 2) -> None:
        self.step_fn = step_fn
        self.warmup = warmup
        self.n = 0
        self.graph: torch.cuda.CUDAGraph | None = None
        self.xs: torch.Tensor | None = None
        self.ts: torch.Tensor | None = None
        self.out: torch.Tensor | None = None
        self.failed = False

    def __call__(self, x: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
        if self.failed or (self.graph is None and self.n < self.warmup):
            self.n += 1
            return self.step_fn(x=x, t=t)
        if self.graph is None:
            try:
                self.xs, self.ts = x.clone(), t.clone()
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    self.step_fn(x=self.xs, t=self.ts)
                torch.cuda.current_stream().wait_stream(side)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    self.out = self.step_fn(x=self.xs, t=self.ts)
                self.graph = graph
                logger.info("FlowStepGraph captured (step %d)", self.n)
            except Exception as exc:  # noqa: BLE001 -- correctness first
                logger.warning("FlowStepGraph: capture failed (%s); eager steps", exc)
                self.failed = True
                return self.step_fn(x=x, t=t)
        self.n += 1
        self.xs.copy_(x)
        self.ts.copy_(t)
        self.graph.replay()
        return self.out.clone()


def fuse_flow_graph(model: torch.nn.Module, warmup: int = 2) -> None:
    """Wrap the step closures ``model.diffusion.sample`` receives in
    ``FlowStepGraph`` (src/umic/graph.py:235-253); nothing else changes."""
    diffusion = model.diffusion
    orig_sample = diffusion.sample

    def sample(*args, **kwargs):
        for key in ("step_fn", "unguided_step_fn"):
            if kwargs.get(key) is not None:
                kwargs[key] = FlowStepGraph(kwargs[key], warmup)
        return orig_sample(*args, **kwargs)

    diffusion.sample = sample
    logger.info("fuse_flow_graph: flow ODE step graph runner installed")
