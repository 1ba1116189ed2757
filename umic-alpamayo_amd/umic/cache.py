"""In-place KV cache with the text RoPE fused into the append.

Same API and semantics as the reference's cache (src/umic/cache.py): an
``InplaceLayer`` holds one layer's keys and values in a buffer allocated once
([B, Hkv, capacity, D], from ``InplaceKVCache.from_dynamic``), ``update``
writes new tokens in place instead of concatenating, and ``crop`` only moves
the write pointer.  Returned keys/values are prefix views of the buffer --
contiguous copies for single-token steps and in graph mode, where the write
goes to a device-held position (replay-safe) and the exact graph length is
returned.

What this build adds is ``InplaceLayer.append_rotary``: the attention's
``apply_rotary_pos_emb`` and ``update`` in ONE gfx950 launch
(``umic_rope_kv_append_bf16``) that rotates q, rotates k straight into the
cache buffer and copies v beside it -- no rotated-k temporary, no separate
copy kernels.  ``umic.integrate.fuse_kv_rope`` routes the text attention
modules through it whenever their cache is an ``InplaceKVCache``.
"""

from __future__ import annotations

import logging

import torch
from transformers.cache_utils import DynamicCache, DynamicLayer

from umic.kernels import rope

logger = logging.getLogger(__name__)


class InplaceLayer(DynamicLayer):
    """One layer's KV in a pre-allocated buffer; appends are copy-free.

    Follows src/umic/cache.py:25-91.  ``keys``/``values`` are strided prefix
    views of the buffers (no ``.contiguous()`` on the multi-token path: that
    would re-copy the prefix).
    """

    def __init__(self, k_buf: torch.Tensor, v_buf: torch.Tensor, base_len: int) -> None:
        super().__init__()
        if k_buf.shape != v_buf.shape or k_buf.dim() != 4:
            raise ValueError(f"InplaceLayer: k/v buffers must be [B,H,L,D] of one shape, got "
                             f"{tuple(k_buf.shape)} and {tuple(v_buf.shape)}")
        if not 0 <= base_len <= k_buf.shape[2]:
            raise ValueError(f"InplaceLayer: base_len {base_len} outside the buffer "
                             f"({k_buf.shape[2]})")
        self._k_buf = k_buf
        self._v_buf = v_buf
        self._pos = base_len
        self.keys = k_buf[:, :, :base_len, :]
        self.values = v_buf[:, :, :base_len, :]
        self.dtype, self.device = k_buf.dtype, k_buf.device
        self.is_initialized = True
        # the buffers never change: check once whether the fused append can
        # write them, per call only the inputs (a missing library then raises
        # at the launch, as every fused path does)
        self._fused_ok = rope.kv_cache_ok(k_buf, v_buf)
        # Graph mode (set by a decode-graph runner): single-token writes go to
        # the device position _pos_t, and the first _graph_len rows are
        # returned, so every replay sees one static shape.
        self.graph_mode = False
        self._pos_t: torch.Tensor | None = None
        self._graph_len = 0

    @property
    def capacity(self) -> int:
        return self._k_buf.shape[2]

    def _graph_write(self, n: int) -> bool:
        return self.graph_mode and n == 1 and self._pos_t is not None

    def _graph_views(self) -> tuple[torch.Tensor, torch.Tensor]:
        self.keys = self._k_buf[:, :, :self._graph_len, :].contiguous()
        self.values = self._v_buf[:, :, :self._graph_len, :].contiguous()
        return self.keys, self.values

    def _advance(self, n: int) -> tuple[torch.Tensor, torch.Tensor]:
        self._pos += n
        self.keys = self._k_buf[:, :, :self._pos, :]
        self.values = self._v_buf[:, :, :self._pos, :]
        if n == 1:
            # single-token steps hand attention contiguous KV (the reference
            # measured strided views slower for the decode GEMV/flash path)
            return self.keys.contiguous(), self.values.contiguous()
        return self.keys, self.values

    def _check_room(self, n: int) -> None:
        if self._pos + n > self.capacity:
            raise RuntimeError(f"InplaceLayer overflow: pos {self._pos} + new {n} > "
                               f"buffer {self.capacity}")

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """Append already-rotated keys and values (src/umic/cache.py:50-80)."""
        n = key_states.shape[2]
        if self._graph_write(n):
            self._k_buf.index_copy_(2, self._pos_t, key_states)
            self._v_buf.index_copy_(2, self._pos_t, value_states)
            return self._graph_views()
        self._check_room(n)
        self._k_buf[:, :, self._pos:self._pos + n, :] = key_states
        self._v_buf[:, :, self._pos:self._pos + n, :] = value_states
        return self._advance(n)

    def can_append_rotary(self, q, k, v, cos, sin, norm=None) -> bool:
        """True when ``append_rotary`` takes its one-launch fused path."""
        return (self._fused_ok and rope.kv_inputs_ok(q, k, v, cos, sin, self._k_buf)
                and (norm is None or rope.norm_weights_ok(q, norm[0], norm[1])))

    def append_rotary(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      cos: torch.Tensor, sin: torch.Tensor, norm=None):
        """rope(q), and the cache after appending rope(k) and v, in one launch.

        Equivalent to ``apply_rotary_pos_emb(q, k, cos, sin)`` followed by
        ``update(k_rot, v)`` (bit for bit: the kernel's rotation is the eager
        bf16 chain's); returns ``(q_rot, keys, values)`` with ``update``'s
        return conventions, or None -- nothing done -- when the inputs are not
        a layout the kernel takes (``can_append_rotary``).  With
        ``norm = (q_w, k_w, eps)``, q and k are the raw projections and the
        attention's per-head RMSNorms (HF q_norm / k_norm) run first, in the
        same launch.
        """
        if not self.can_append_rotary(q, k, v, cos, sin, norm):
            return None
        n = k.shape[2]
        if self._graph_write(n):
            if not (self._pos_t.dtype == torch.int64 and self._pos_t.device == self.device):
                return None
            q_rot = rope.kv_launch(q, k, v, cos, sin, self._k_buf, self._v_buf, 0, self._pos_t,
                                   norm)
            return (q_rot, *self._graph_views())
        self._check_room(n)
        q_rot = rope.kv_launch(q, k, v, cos, sin, self._k_buf, self._v_buf, self._pos, None, norm)
        return (q_rot, *self._advance(n))

    def get_seq_length(self, cache_position=None) -> int:
        return self._pos

    def get_max_length(self) -> int:
        return self.capacity

    def crop(self, max_length: int) -> None:
        """O(1): move the write pointer back (negative = drop that many)."""
        if max_length < 0:
            max_length = self._pos + max_length
        self._pos = max(0, min(self._pos, max_length))
        self.keys = self._k_buf[:, :, :self._pos, :]
        self.values = self._v_buf[:, :, :self._pos, :]


class InplaceKVCache(DynamicCache):
    """DynamicCache whose layers are pre-allocated ``InplaceLayer`` s.

    Subclassing DynamicCache keeps transformers' mask and attention back-end
    selection identical (src/umic/cache.py:94-160).
    """

    def __init__(self, layers: list[InplaceLayer]) -> None:
        super().__init__()
        self.layers = layers

    @classmethod
    def from_dynamic(cls, cache: DynamicCache, extra_tokens: int,
                     margin: int = 8) -> "InplaceKVCache":
        """Convert once: allocate base_len + extra_tokens + margin rows per
        layer and copy the existing prefix (src/umic/cache.py:104-128)."""
        layers: list[InplaceLayer] = []
        alloc = 0
        for lyr in cache.layers:
            k, v = lyr.keys, lyr.values
            b, h, base_len, d = k.shape
            kb = torch.empty(b, h, base_len + extra_tokens + margin, d, device=k.device,
                             dtype=k.dtype)
            vb = torch.empty_like(kb)
            kb[:, :, :base_len, :] = k
            vb[:, :, :base_len, :] = v
            layers.append(InplaceLayer(kb, vb, base_len))
            alloc += kb.numel() * kb.element_size() * 2
        logger.info("InplaceKVCache: %d layers converted, base_len=%d, alloc=%.0f MB",
                    len(layers), layers[0]._pos if layers else 0, alloc / 1e6)
        return cls(layers)

    def crop(self, max_length: int) -> None:
        for lyr in self.layers:
            lyr.crop(max_length)

    # --- graph-mode plumbing (driven by a decode-graph runner) -------------

    def enable_graph_mode(self, pos_t: torch.Tensor) -> None:
        """Static-shape decode: writes at device position pos_t, full reads."""
        for lyr in self.layers:
            lyr.graph_mode = True
            lyr._pos_t = pos_t

    def disable_graph_mode(self) -> None:
        for lyr in self.layers:
            lyr.graph_mode = False
            lyr.keys = lyr._k_buf[:, :, :lyr._pos, :]
            lyr.values = lyr._v_buf[:, :, :lyr._pos, :]

    def set_pos(self, n: int) -> None:
        """Sync the host write pointer after graph replays."""
        for lyr in self.layers:
            lyr._pos = n

    def set_graph_len(self, n: int) -> None:
        """Exact KV length for the graph being captured / replayed."""
        for lyr in self.layers:
            lyr._graph_len = n

    def get_seq_length(self, layer_idx: int = 0, cache_position=None) -> int:
        if layer_idx >= len(self.layers):
            return 0
        return self.layers[layer_idx].get_seq_length()
