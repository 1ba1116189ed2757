"""HIP graphs for the two repeated steps of a UMIC inference: generate()'s
single-token decode and the flow expert's ODE step.

Both replay captured work on static buffers; what differs is the key.

* Decode (``DecodeGraphRunner``): one graph per KV length.  Attention over
  an exact-length cache keeps attention_mask=None and so the fused SDPA
  kernels with grouped-query heads; a padded single graph would need a 4-D
  mask (the reference measured that slower, src/umic/graph.py:11-14).  The
  runner owns a persistent ``InplaceKVCache``: a new inference with the same
  prompt length is re-seeded into the same buffers, so graphs captured
  earlier stay valid and later inferences are pure replay.  Every replay
  writes its KV row at the arena's device cursor; with
  ``umic.integrate.fuse_kv_rope`` each layer's q_norm, k_norm, RoPE and append
  inside the graph is one ``umic_qk_rmsnorm_rope_kv_append_bf16`` launch.
* Flow (``FlowStepGraph``): the ODE step runs on fixed shapes -- its action
  tokens are appended to the prefix cache at the same rows and cropped back
  -- so one graph serves every step; only the values of x and t change.

Capture never decides results: a step that cannot be captured runs eagerly.
"""

from __future__ import annotations

import functools
import gc
import logging
from typing import Any, Callable

import torch
from transformers.cache_utils import DynamicCache

from umic.cache import InplaceKVCache

logger = logging.getLogger(__name__)


def _on_side_stream(fn: Callable[[], Any]):
    """Run fn on a side stream ordered after the current one (allocator and
    library lazy initialisation must not land inside a later capture: the
    torch.cuda.graphs warm-up recipe)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = fn()
    torch.cuda.current_stream().wait_stream(side)
    return out


def _capture(fn: Callable[[], Any], pool=None, warm: bool = True):
    """Capture one call of fn in a new graph, after one warm-up call on a
    side stream unless ``warm`` is False; returns (graph, outputs).

    Python's cyclic garbage collector is held off while the capture is open.
    A collection there finalizes whatever dead cycles exist at that moment --
    a discarded runner is one (the model's forward holds the runner, which
    holds the model) -- and so can destroy their graphs and release their
    graph memory pools inside another stream capture; a test process once
    aborted during such a collection.  torch.cuda.graph no longer collects
    before a capture by default, so the guard is here."""
    if warm:
        _on_side_stream(fn)
    graph = torch.cuda.CUDAGraph()
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph, pool=pool):
            out = fn()
    finally:
        if was_enabled:
            gc.enable()
    return graph, out


class _GraphBank:
    """Captured steps keyed by KV length, sharing one memory pool."""

    def __init__(self) -> None:
        self._steps: dict[int, tuple[torch.cuda.CUDAGraph, Any]] = {}
        self._pool = None

    def __len__(self) -> int:
        return len(self._steps)

    def __contains__(self, key: int) -> bool:
        return key in self._steps

    def run(self, key: int, fn: Callable[[], Any], warm: bool):
        """Replay the step for key, capturing it first if needed; its outputs."""
        if key not in self._steps:
            graph, out = _capture(fn, self._pool, warm)
            if self._pool is None:
                self._pool = graph.pool()
            self._steps[key] = (graph, out)
        graph, out = self._steps[key]
        graph.replay()
        return out

    def clear(self) -> None:
        self._steps.clear()
        self._pool = None


class _StepIO:
    """Static device inputs of the captured decode step: the token, the
    position ids (the form generate() passes, or None), the model's M-RoPE
    delta and the arena write cursor."""

    def __init__(self, device, pids: torch.Tensor | None) -> None:
        self.ids = torch.zeros(1, 1, dtype=torch.long, device=device)
        self.cursor = torch.zeros(1, dtype=torch.long, device=device)
        self.delta = torch.zeros(1, dtype=torch.long, device=device)
        self.pids = None if pids is None else torch.zeros_like(pids)

    def matches(self, pids: torch.Tensor | None) -> bool:
        if (pids is None) != (self.pids is None):
            return False
        return pids is None or (pids.shape == self.pids.shape and pids.dtype == self.pids.dtype)

    def load(self, ids: torch.Tensor, pids: torch.Tensor | None, pos: int) -> None:
        self.ids.copy_(ids)
        self.cursor.fill_(pos)
        if pids is not None:
            self.pids.copy_(pids)

    def position_ids(self) -> torch.Tensor:
        if self.pids is not None:
            return self.pids
        # no ids given: text position + the model's rope delta on all three
        # M-RoPE rows (src/umic/graph.py:128-136)
        return (self.cursor + self.delta).view(1, 1, 1).expand(3, 1, 1)


# forward() arguments that carry new multimodal input or replace input_ids
_MULTIMODAL = ("inputs_embeds", "pixel_values", "pixel_values_videos")
# arguments the captured step supplies itself
_STEP_ARGS = ("input_ids", "attention_mask", "past_key_values", "position_ids", "cache_position")


class DecodeGraphRunner:
    """Installs itself as the VLM's forward and serves generate()'s
    single-token decode steps from per-KV-length graphs (public contract of
    src/umic/graph.py:36-176: persistent buffers, a re-seed per inference,
    sampling left eager between replays).  Every other call -- prefill,
    multimodal input, padded prompts, CPU tensors -- runs the model's own
    forward."""

    def __init__(self, vlm: torch.nn.Module, max_new_tokens: int = 96,
                 warmup_steps: int = 2) -> None:
        self.vlm = vlm
        self.max_new = max_new_tokens
        self.warmup_steps = warmup_steps
        self.replays = 0
        self._model_forward = vlm.forward
        self._bank = _GraphBank()
        self._kv: InplaceKVCache | None = None     # persistent arena cache
        self._kv_prompt: int | None = None         # prompt length it was built for
        self._io: _StepIO | None = None
        self._step_kwargs: dict[str, Any] = {}
        self._eager_steps = 0
        self._live = False                          # inside a decode session on _kv
        self._off = False                           # a capture failed: eager for good

        @functools.wraps(self._model_forward)
        def forward(*args: Any, **kwargs: Any):
            return self._dispatch(args, kwargs)

        forward._umic_runner = self
        vlm.forward = forward
        generate = getattr(vlm, "generate", None)
        if generate is not None:
            @functools.wraps(generate)
            def generate_and_release(*args: Any, **kwargs: Any):
                try:
                    return generate(*args, **kwargs)
                finally:
                    self._close()

            vlm.generate = generate_and_release
        logger.info("decode graph runner installed on %s", type(vlm).__name__)

    # public views of the runner's state
    @property
    def graphs(self) -> _GraphBank:
        return self._bank

    @property
    def cache(self) -> InplaceKVCache | None:
        return self._kv

    @property
    def wrapped_forward(self):
        """The model forward the runner dispatches to."""
        return self._model_forward

    # -- session bookkeeping -----------------------------------------------

    def _close(self) -> None:
        """A generate() returned (or a step went eager): host-positioned writes
        again, so the cache is an ordinary in-place cache for later users."""
        if self._kv is not None:
            self._kv.end_replay()
        self._live = False
        self._eager_steps = 0

    def _is_step(self, args, kwargs) -> bool:
        ids, pkv = kwargs.get("input_ids"), kwargs.get("past_key_values")
        return (not args and not self._off and isinstance(ids, torch.Tensor) and ids.is_cuda
                and tuple(ids.shape) == (1, 1) and isinstance(pkv, DynamicCache)
                and pkv.get_seq_length() > 0
                and all(kwargs.get(name) is None for name in _MULTIMODAL)
                and not torch.cuda.is_current_stream_capturing())

    def _open(self, kwargs: dict[str, Any]) -> bool:
        """First decode step of a generate(): move its cache into the arena."""
        pkv = kwargs["past_key_values"]
        if any(getattr(lyr, "keys", None) is None for lyr in pkv.layers):
            return False
        mask = kwargs.get("attention_mask")
        if mask is not None and not bool((mask == 1).all().item()):
            logger.warning("decode graph runner: padded prompt, decoding eagerly")
            return False
        prompt = pkv.get_seq_length()
        if pkv is not self._kv:
            if self._kv is not None and prompt == self._kv_prompt:
                self._kv.reseed(pkv)             # same buffers: graphs stay valid
            else:
                if self._kv is not None:
                    logger.info("decode graph runner: prompt %s -> %d tokens, new graphs",
                                self._kv_prompt, prompt)
                self._bank.clear()
                self._kv = InplaceKVCache.from_dynamic(pkv, extra_tokens=self.max_new)
                self._kv_prompt = prompt
        pids = kwargs.get("position_ids")
        if self._io is None or not self._io.matches(pids):
            self._bank.clear()                   # the step's inputs change form
            self._io = _StepIO(kwargs["input_ids"].device, pids)
        delta = getattr(getattr(self.vlm, "model", None), "rope_deltas", None)
        if isinstance(delta, torch.Tensor):
            self._io.delta.copy_(delta.reshape(-1)[:1])
        else:
            self._io.delta.zero_()
        self._step_kwargs = {k: v for k, v in kwargs.items() if k not in _STEP_ARGS}
        self._live = True
        return True

    # -- the step ----------------------------------------------------------

    def _static_step(self):
        io = self._io
        return self._model_forward(input_ids=io.ids, attention_mask=None,
                                   past_key_values=self._kv, position_ids=io.position_ids(),
                                   **self._step_kwargs)

    def _eager(self, args, kwargs):
        if self._live and kwargs.get("past_key_values") is self._kv:
            self._close()                        # appends at the host position
        return self._model_forward(*args, **kwargs)

    def _dispatch(self, args, kwargs):
        if not self._is_step(args, kwargs):
            return self._eager(args, kwargs)
        if (not self._live or kwargs["past_key_values"] is not self._kv) and \
                not self._open(kwargs):
            return self._eager(args, kwargs)
        if not self._io.matches(kwargs.get("position_ids")):
            return self._eager(args, kwargs)
        pos = self._kv.get_seq_length()          # tokens held (host)
        if pos + 1 > self._kv.layers[0].capacity:
            raise RuntimeError(f"decode graph runner: step {pos + 1 - self._kv_prompt} is past "
                               f"the cache headroom (max_new_tokens={self.max_new})")
        self._io.load(kwargs["input_ids"], kwargs.get("position_ids"), pos)
        self._kv.replay_at(self._io.cursor, pos + 1)
        if not len(self._bank) and self._eager_steps < self.warmup_steps:
            # the first steps of a runner's life run the static step eagerly
            # (library lazy initialisation happens outside any capture)
            self._eager_steps += 1
            out = _on_side_stream(self._static_step)
        else:
            try:
                out = self._bank.run(pos + 1, self._static_step, warm=False)
            except Exception as exc:  # noqa: BLE001 -- results never depend on capture
                logger.warning("decode graph runner: capture failed (%s), decoding eagerly", exc)
                self._off = True
                self._kv.set_length(pos)
                return self._eager(args, kwargs)
            self.replays += 1
        self._kv.set_length(pos + 1)
        return out


def fuse_decode_graph(vlm: torch.nn.Module, max_new_tokens: int = 96) -> DecodeGraphRunner:
    """Install the per-length decode graph runner on the VLM
    (src/umic/graph.py:179-181).  Idempotent: a VLM that already carries a
    runner keeps it, with the larger headroom."""
    existing = getattr(getattr(vlm, "forward", None), "_umic_runner", None)
    if isinstance(existing, DecodeGraphRunner):
        existing.max_new = max(existing.max_new, max_new_tokens)
        return existing
    return DecodeGraphRunner(vlm, max_new_tokens=max_new_tokens)


class FlowStepGraph:
    """``step_fn(x=, t=)`` served from one graph after ``warmup`` eager calls
    (contract of src/umic/graph.py:179-232).  The graph holds the addresses of
    the cache it was captured on: one instance per inference."""

    def __init__(self, step_fn, warmup: int = 2) -> None:
        self.step_fn = step_fn
        self.warmup = warmup
        self.calls = 0
        self._graph: torch.cuda.CUDAGraph | None = None
        self._xt: tuple[torch.Tensor, torch.Tensor] | None = None
        self._out: torch.Tensor | None = None
        self._off = False

    @property
    def captured(self) -> bool:
        return self._graph is not None

    @property
    def disabled(self) -> bool:
        """A capture failed: every later step runs eagerly."""
        return self._off

    def _try_capture(self, x: torch.Tensor, t: torch.Tensor) -> bool:
        xs, ts = x.clone(), t.clone()
        try:
            graph, out = _capture(lambda: self.step_fn(x=xs, t=ts))
        except Exception as exc:  # noqa: BLE001 -- results never depend on capture
            logger.warning("flow step graph: capture failed (%s), eager steps", exc)
            self._off = True
            return False
        self._graph, self._xt, self._out = graph, (xs, ts), out
        logger.info("flow step graph captured at call %d", self.calls)
        return True

    def __call__(self, x: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
        self.calls += 1
        if self._graph is None and (self._off or self.calls <= self.warmup
                                    or not self._try_capture(x, t)):
            return self.step_fn(x=x, t=t)
        self._xt[0].copy_(x)
        self._xt[1].copy_(t)
        self._graph.replay()
        return self._out.clone()


_FLOW_STEP_KWARGS = ("step_fn", "unguided_step_fn")


def fuse_flow_graph(model: torch.nn.Module, warmup: int = 2) -> None:
    """Serve the flow expert's ODE steps from graphs: the step closures that
    ``model.diffusion.sample`` receives are wrapped in ``FlowStepGraph``
    (src/umic/graph.py:235-253)."""
    sample = model.diffusion.sample

    @functools.wraps(sample)
    def sample_with_graphs(*args, **kwargs):
        for name in _FLOW_STEP_KWARGS:
            if kwargs.get(name) is not None:
                kwargs[name] = FlowStepGraph(kwargs[name], warmup)
        return sample(*args, **kwargs)

    model.diffusion.sample = sample_with_graphs
    logger.info("fuse_flow_graph: flow ODE step graphs installed")
