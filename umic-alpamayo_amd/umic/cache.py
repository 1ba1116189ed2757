"""In-place KV cache for repeated decode / flow steps, written by the fused
RoPE + append kernel.

Storage.  A ``KVArena`` is one device allocation holding every layer's keys
and values, ``[layers, 2, batch, kv_heads, capacity, head_dim]``: each
layer's k and v are adjacent views with identical strides (what the fused
append kernel writes), and converting or re-seeding a cache is one copy per
layer into memory that never moves.  The arena keeps each layer's fill level
on the host, and -- for graph replay -- one device int64 write cursor and
one attention window shared by all layers: a replayed single-token step
writes its row at the cursor and hands attention exactly ``window`` rows.

Writes.  ``InplaceLayer.append_rotary(q, k, v, cos, sin, norm)`` is the
primary path: one launch rotates q, rotates k straight into the layer's key
rows, copies v beside it, and (with ``norm``) applies the attention's q_norm /
k_norm first (``umic_qk_rmsnorm_rope_kv_append_bf16``); under replay it
writes at the arena cursor.  ``update(k, v)`` takes already-rotated keys --
the interface transformers' attention calls -- and writes the same rows.

Observable behaviour is the reference's in-place cache
(src/umic/cache.py:25-160), which this replaces: keys/values are the
prefix of the buffer (strided views; single-token steps and replays return
contiguous copies), ``crop`` is O(1), a write past the capacity raises
instead of growing, and ``InplaceKVCache`` is a transformers DynamicCache,
so mask and attention back-end selection are unchanged.
"""

from __future__ import annotations

import weakref

import torch
from transformers.cache_utils import DynamicCache, DynamicLayer

from umic import _lib
from umic.kernels import rope


class KVArena:
    """Keys and values of ``layers`` layers in one allocation.

    ``fill[i]`` tokens of layer i are valid (rows 0 .. fill[i] - 1).  While
    ``cursor`` is set (a device int64 [1] tensor) single-token writes go to
    row ``cursor`` and attention sees ``window`` rows.
    """

    def __init__(self, layers: int, batch: int, heads: int, capacity: int, head_dim: int,
                 dtype: torch.dtype, device: torch.device | str) -> None:
        if min(layers, batch, heads, head_dim) <= 0 or capacity < 0:
            raise ValueError(f"KVArena: bad geometry layers={layers} batch={batch} "
                             f"heads={heads} capacity={capacity} head_dim={head_dim}")
        self.storage = torch.empty(layers, 2, batch, heads, capacity, head_dim, dtype=dtype,
                                   device=device)
        self.fill = [0] * layers
        self.cursor: torch.Tensor | None = None
        self.window = 0
        # the buffers never move: check once whether the fused append can write them
        self.fused_ok = rope.kv_cache_ok(self.k(0), self.v(0)) and _lib.available()

    @property
    def capacity(self) -> int:
        return self.storage.shape[4]

    @property
    def layers(self) -> int:
        return self.storage.shape[0]

    def k(self, i: int) -> torch.Tensor:
        return self.storage[i, 0]

    def v(self, i: int) -> torch.Tensor:
        return self.storage[i, 1]

    def rows(self, i: int, n: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Views of layer i's first n rows."""
        return self.storage[i, 0, :, :, :n], self.storage[i, 1, :, :, :n]

    def room(self, i: int, n: int) -> int:
        """Row where n new tokens of layer i go; raises if they do not fit."""
        start = self.fill[i]
        if start + n > self.capacity:
            raise RuntimeError(f"KV arena overflow (layer {i}): {start} tokens held + {n} new "
                               f"> capacity {self.capacity}")
        return start

    def replaying(self, n: int) -> bool:
        return self.cursor is not None and n == 1


class InplaceLayer(DynamicLayer):
    """Layer ``index`` of an arena with transformers' DynamicLayer interface.

    ``keys`` / ``values`` are refreshed after every operation: views of the
    valid rows, contiguous copies for single-token steps and replays.
    """

    def __init__(self, arena: KVArena, index: int) -> None:
        super().__init__()
        self.arena, self.index = arena, index
        self.dtype, self.device = arena.storage.dtype, arena.storage.device
        self.is_initialized = True
        self._views()

    @property
    def capacity(self) -> int:
        return self.arena.capacity

    def _views(self, n: int | None = None, copy: bool = False):
        n = self.arena.fill[self.index] if n is None else n
        k, v = self.arena.rows(self.index, n)
        if copy:
            k, v = k.contiguous(), v.contiguous()
        self.keys, self.values = k, v
        return k, v

    def _wrote(self, n: int):
        """Bookkeeping after writing n tokens: the new views."""
        ar = self.arena
        if ar.replaying(n):
            return self._views(ar.window, copy=True)
        ar.fill[self.index] += n
        # single-token steps hand attention contiguous KV (the reference
        # measured strided views slower for the decode attention kernels)
        return self._views(copy=n == 1)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """Append already-rotated keys and their values (src/umic/cache.py:50-80)."""
        ar, i, n = self.arena, self.index, key_states.shape[2]
        if ar.replaying(n):
            ar.k(i).index_copy_(2, ar.cursor, key_states)
            ar.v(i).index_copy_(2, ar.cursor, value_states)
        else:
            r0 = ar.room(i, n)
            ar.k(i)[:, :, r0:r0 + n] = key_states
            ar.v(i)[:, :, r0:r0 + n] = value_states
        return self._wrote(n)

    def can_append_rotary(self, q, k, v, cos, sin, norm=None) -> bool:
        """True when ``append_rotary`` takes its one-launch fused path."""
        ar = self.arena
        if not (ar.fused_ok and rope.kv_inputs_ok(q, k, v, cos, sin, ar.k(self.index))):
            return False
        if norm is not None and not rope.norm_weights_ok(q, norm[0], norm[1]):
            return False
        if ar.replaying(k.shape[2]):
            c = ar.cursor
            return c.dtype == torch.int64 and c.device == self.device
        return True

    def append_rotary(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      cos: torch.Tensor, sin: torch.Tensor, norm=None):
        """rope(q), and the layer's keys and values after appending rope(k) and
        v, in one launch: ``(q_rot, keys, values)`` with ``update``'s return
        conventions, or None -- nothing done -- for inputs the kernel does not
        take.  Bit for bit ``apply_rotary_pos_emb(q, k, cos, sin)`` followed by
        ``update``.  With ``norm = (q_w, k_w, eps)`` q and k are the raw
        projections and the attention's q_norm / k_norm run first, in the
        same launch."""
        if not self.can_append_rotary(q, k, v, cos, sin, norm):
            return None
        ar, i, n = self.arena, self.index, k.shape[2]
        if ar.replaying(n):
            q_rot = rope.kv_launch(q, k, v, cos, sin, ar.k(i), ar.v(i), 0, ar.cursor, norm)
        else:
            q_rot = rope.kv_launch(q, k, v, cos, sin, ar.k(i), ar.v(i), ar.room(i, n), None,
                                   norm)
        return (q_rot, *self._wrote(n))

    def get_seq_length(self, cache_position=None) -> int:
        return self.arena.fill[self.index]

    def get_max_length(self) -> int:
        return self.arena.capacity

    def crop(self, max_length: int) -> None:
        """O(1): keep max_length tokens (a negative value drops that many)."""
        held = self.arena.fill[self.index]
        keep = held + max_length if max_length < 0 else max_length
        self.arena.fill[self.index] = max(0, min(held, keep))
        self._views()


class InplaceKVCache(DynamicCache):
    """A DynamicCache whose layers are views of ``KVArena`` s."""

    def __init__(self, layers: list[InplaceLayer]) -> None:
        super().__init__()
        self.layers = layers
        self.arenas = list({id(lyr.arena): lyr.arena for lyr in layers}.values())

    @classmethod
    def from_dynamic(cls, cache: DynamicCache, extra_tokens: int,
                     margin: int = 8) -> "InplaceKVCache":
        """Copy a populated cache into an arena with room for extra_tokens
        (+ margin) more tokens per layer.  Layers of one geometry share one
        arena; any other layer gets its own."""
        layers: list[InplaceLayer] = []
        arenas: dict[tuple, tuple[KVArena, list[int]]] = {}
        for idx, lyr in enumerate(cache.layers):
            k = lyr.keys
            key = (tuple(k.shape[:2]), k.shape[3], k.shape[2], k.dtype, str(k.device))
            arenas.setdefault(key, (None, []))[1].append(idx)
        slot: dict[int, tuple[KVArena, int]] = {}
        for (bh, d, held, dt, dev), (_, members) in arenas.items():
            ar = KVArena(len(members), bh[0], bh[1], held + extra_tokens + margin, d, dt, dev)
            for j, idx in enumerate(members):
                src = cache.layers[idx]
                ar.storage[j, 0, :, :, :held].copy_(src.keys)
                ar.storage[j, 1, :, :, :held].copy_(src.values)
                ar.fill[j] = held
                slot[idx] = (ar, j)
        for idx in range(len(cache.layers)):
            layers.append(InplaceLayer(*slot[idx]))
        return cls(layers)

    def reseed(self, cache: DynamicCache) -> None:
        """Copy another cache's contents (same geometry, at most the capacity)
        into these buffers, in place: captured graphs keep valid addresses."""
        for dst, src in zip(self.layers, cache.layers):
            n = src.keys.shape[2]
            k, v = dst.arena.rows(dst.index, n)
            k.copy_(src.keys)
            v.copy_(src.values)
            dst.arena.fill[dst.index] = n
            dst._views()

    def crop(self, max_length: int) -> None:
        for lyr in self.layers:
            lyr.crop(max_length)

    # -- graph replay --------------------------------------------------------

    def replay_at(self, cursor: torch.Tensor, window: int) -> None:
        """Single-token writes go to device row ``cursor``; attention sees
        ``window`` rows (the KV length the replayed graph was captured at)."""
        for ar in self.arenas:
            ar.cursor, ar.window = cursor, window

    def end_replay(self) -> None:
        """Back to host-positioned writes at each layer's fill level."""
        for ar in self.arenas:
            ar.cursor = None
        for lyr in self.layers:
            lyr._views()

    def set_length(self, n: int) -> None:
        """Every layer holds n tokens (after replays wrote them on the device)."""
        for lyr in self.layers:
            lyr.arena.fill[lyr.index] = n
            if lyr.arena.cursor is None:
                lyr._views()

    def get_seq_length(self, layer_idx: int = 0, cache_position=None) -> int:
        if layer_idx >= len(self.layers):
            return 0
        return self.layers[layer_idx].get_seq_length()


class CacheStandIn:
    """The ``InplaceKVCache`` that stands in for a caller's ``DynamicCache``
    across the calls of an append-then-crop loop (a flow expert's denoising
    steps, a decode loop).

    The caller keeps its own cache and crops it back to the prefix after
    every step.  ``resolve(source, n_new)`` returns the stand-in for
    ``source``: built (one copy into an arena with room for the step's new
    tokens) the first time that cache object is seen, and thereafter only
    cut back to ``source``'s length, an O(1) crop that makes the caller's
    own crop redundant.  The source is held by a weak reference and compared
    by identity, so a later cache -- even one CPython places at a freed
    cache's address -- is never mistaken for the one converted before.
    ``None`` means "leave the call alone": no cache, a stand-in already, or
    a cache whose layers are not all populated yet (generate() creates
    them empty before prefill).
    """

    def __init__(self, extra_tokens: int = 64) -> None:
        self.extra_tokens = extra_tokens
        self._source: weakref.ref | None = None
        self._inplace: InplaceKVCache | None = None

    @staticmethod
    def convertible(cache) -> bool:
        if not isinstance(cache, DynamicCache) or isinstance(cache, InplaceKVCache):
            return False
        layers = getattr(cache, "layers", None)
        return bool(layers) and all(getattr(lyr, "keys", None) is not None for lyr in layers)

    def bound_to(self, cache) -> bool:
        return self._source is not None and self._source() is cache

    def resolve(self, source, n_new: int = 0) -> "InplaceKVCache | None":
        if not self.convertible(source):
            return None
        if not self.bound_to(source):
            self._inplace = InplaceKVCache.from_dynamic(
                source, extra_tokens=max(n_new, self.extra_tokens))
            self._source = weakref.ref(source)
        self._inplace.crop(source.get_seq_length())
        return self._inplace
