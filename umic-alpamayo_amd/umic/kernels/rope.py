"""Fused rotary embedding of q and k on gfx950 (libumic_hip.so).

Drop-in for the reference's RoPE wrappers (src/umic/kernels/rope.py):
``apply_rotary_vision_hip`` replaces ``apply_rotary_vision_triton`` (:78-84,
signature of HF ``apply_rotary_pos_emb_vision``) and ``make_text_rope`` (:86-107)
builds the replacement for HF ``apply_rotary_pos_emb``.  Unlike the reference,
q and k are rotated in ONE launch that reads cos/sin once.

Numerics are the eager HF functions' own:
  text    (modeling_qwen3_vl.py:412-435)  every op in bf16 --
          bf16(bf16(q*cos) + bf16(rotate_half(q)*sin)), cos/sin bf16;
  vision  (modeling_qwen3_vl.py:145-156)  q.float(), fp32 cos/sin, products
          and sum each rounded in fp32, one final cast to bf16.
Outputs are allocated like eager's: ``torch.empty_like`` keeps a dense input's
strides (so a transposed [B,H,S,D] view of [B,S,H,D] stays in that layout)
and gives a contiguous tensor for a strided view such as q/k of a packed qkv.
"""

from __future__ import annotations

import inspect

import torch

from umic import _lib
from umic.kernels._common import grad_needed, require_device

MAX_HEAD_DIM = 1024  # cos/sin rows of a block's positions are staged in LDS


def _strides_bsh(t: torch.Tensor, order: str) -> tuple[int, int, int]:
    """(batch, position, head) element strides of t laid out as `order`."""
    if order == "bhsd":
        return t.stride(0), t.stride(2), t.stride(1)
    if order == "shd":
        return 0, t.stride(0), t.stride(1)
    raise ValueError(order)


def _rope(q, k, cos, sin, mode: int, order: str) -> tuple[torch.Tensor, torch.Tensor]:
    if order == "bhsd":
        B, Hq, S, D = q.shape
        Hk = k.shape[1]
        cs_sb = cos.stride(0) if cos.shape[0] == B else 0
        cs_ss = cos.stride(1)
    else:
        S, Hq, D = q.shape
        B, Hk = 1, k.shape[1]
        cs_sb, cs_ss = 0, cos.stride(0)
    q_out, k_out = torch.empty_like(q), torch.empty_like(k)
    qs, ks = _strides_bsh(q, order), _strides_bsh(k, order)
    qos, kos = _strides_bsh(q_out, order), _strides_bsh(k_out, order)
    with _lib.device_of(q):
        _lib.call("umic_rope_qk_bf16", q.data_ptr(), k.data_ptr(), q_out.data_ptr(),
                  k_out.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                  int(cos.dtype == torch.float32), mode, B, S, Hq, Hk, D,
                  *qs, *ks, *qos, *kos, cs_sb, cs_ss, _lib.stream_of(q))
    return q_out, k_out


def _same_table_layout(cos: torch.Tensor, sin: torch.Tensor) -> bool:
    return (cos.shape == sin.shape and cos.stride() == sin.stride() and cos.dtype == sin.dtype
            and cos.device == sin.device and cos.stride(-1) == 1)


def text_rope_eligible(q, k, cos, sin, unsqueeze_dim=1) -> bool:
    """HF text layout the kernel reproduces exactly: q/k [B,H,S,D] bf16 on the
    GPU, cos/sin [B or 1, S, D] bf16, broadcast over heads (unsqueeze_dim 1)."""
    if unsqueeze_dim != 1 or not all(isinstance(t, torch.Tensor) for t in (q, k, cos, sin)):
        return False
    if not (q.is_cuda and q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16
            and cos.dtype == torch.bfloat16 and q.dim() == 4 and k.dim() == 4 and cos.dim() == 3):
        return False
    B, _, S, D = q.shape
    return (k.shape[0] == B and k.shape[2] == S and k.shape[3] == D and D % 2 == 0
            and D <= MAX_HEAD_DIM
            and cos.shape[1] == S and cos.shape[2] == D and cos.shape[0] in (1, B)
            and q.stride(-1) == 1 and k.stride(-1) == 1 and _same_table_layout(cos, sin)
            and k.device == q.device and cos.device == q.device)


def vision_rope_eligible(q, k, cos, sin) -> bool:
    """HF vision layout: q/k [S,H,D] bf16 on the GPU, cos/sin [S, D] fp32/bf16."""
    if not all(isinstance(t, torch.Tensor) for t in (q, k, cos, sin)):
        return False
    if not (q.is_cuda and q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16
            and q.dim() == 3 and k.dim() == 3 and cos.dim() == 2
            and cos.dtype in (torch.float32, torch.bfloat16)):
        return False
    S, _, D = q.shape
    return (k.shape[0] == S and k.shape[2] == D and D % 2 == 0 and D <= MAX_HEAD_DIM
            and tuple(cos.shape) == (S, D)
            and q.stride(-1) == 1 and k.stride(-1) == 1 and _same_table_layout(cos, sin)
            and k.device == q.device and cos.device == q.device)


def apply_rotary_text_hip(q, k, cos, sin):
    """HF text RoPE (unsqueeze_dim=1): q [B,Hq,S,D], k [B,Hk,S,D], cos/sin [B,S,D]."""
    require_device(q, k, cos, sin)
    if not text_rope_eligible(q, k, cos, sin):
        raise ValueError("apply_rotary_text_hip: unsupported layout "
                         f"q{tuple(q.shape)} k{tuple(k.shape)} cos{tuple(cos.shape)}")
    return _rope(q, k, cos, sin, _lib.UMIC_ROPE_TEXT, "bhsd")


def apply_rotary_vision_hip(q, k, cos, sin):
    """Drop-in for HF apply_rotary_pos_emb_vision (q/k: [S, H, D])."""
    if not (q.is_cuda and cos.is_cuda):
        raise ValueError("apply_rotary_vision_hip: GPU tensors required")
    require_device(q, k)
    if not vision_rope_eligible(q, k, cos, sin):
        raise ValueError("apply_rotary_vision_hip: unsupported layout "
                         f"q{tuple(q.shape)} k{tuple(k.shape)} cos{tuple(cos.shape)}")
    return _rope(q, k, cos, sin, _lib.UMIC_ROPE_VISION, "shd")


def _unsqueeze_dim_of(fallback):
    """Return f(args, kwargs) -> unsqueeze_dim for calls of `fallback`'s signature.

    transformers 5.x has apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1);
    4.x had a position_ids parameter before it.  Binding against the wrapped
    function's own signature reads the argument correctly in both.
    """
    try:
        sig = inspect.signature(fallback)
    except (TypeError, ValueError):
        sig = None

    def get(args, kwargs):
        if sig is None:
            return kwargs.get("unsqueeze_dim", 1 if not args else None)
        try:
            bound = sig.bind(None, None, None, None, *args, **kwargs)
        except TypeError:
            return None
        bound.apply_defaults()
        return bound.arguments.get("unsqueeze_dim", 1)

    return get


def make_text_rope(fallback):
    """Build a drop-in for HF apply_rotary_pos_emb around `fallback`.

    The HF layout (q/k [B,H,S,D] bf16 on the GPU, cos/sin [B,S,D] bf16,
    unsqueeze_dim 1) runs the fused kernel; every other call -- CPU tensors,
    other dtypes or layouts -- goes to `fallback` with its arguments untouched.
    Any batch size is handled (the reference's fast path required B == 1).
    """
    unsq = _unsqueeze_dim_of(fallback)

    def apply_rotary_text(q, k, cos, sin, *args, **kwargs):
        if (text_rope_eligible(q, k, cos, sin, unsq(args, kwargs))
                and not grad_needed(q, k, cos, sin)):
            require_device(q, k, cos, sin)
            return _rope(q, k, cos, sin, _lib.UMIC_ROPE_TEXT, "bhsd")
        return fallback(q, k, cos, sin, *args, **kwargs)

    apply_rotary_text.__wrapped__ = fallback
    return apply_rotary_text


def make_vision_rope(fallback):
    """Drop-in for HF apply_rotary_pos_emb_vision with an eager fallback."""

    def apply_rotary_vision(q, k, cos, sin, *args, **kwargs):
        if (not args and not kwargs and vision_rope_eligible(q, k, cos, sin)
                and not grad_needed(q, k, cos, sin)):
            require_device(q, k)
            return _rope(q, k, cos, sin, _lib.UMIC_ROPE_VISION, "shd")
        return fallback(q, k, cos, sin, *args, **kwargs)

    apply_rotary_vision.__wrapped__ = fallback
    return apply_rotary_vision


def _vec_ok(*tensors: torch.Tensor) -> bool:
    """16-byte chunks: unit inner stride, the other strides multiples of 8
    elements, 16-byte aligned data."""
    for t in tensors:
        st = t.stride()
        if st[-1] != 1 or t.data_ptr() % 16:
            return False
        for s in st[:-1]:
            if s % 8:
                return False
    return True


def kv_cache_ok(k_cache: torch.Tensor, v_cache: torch.Tensor) -> bool:
    """Cache buffers ``rope_kv_append`` writes: [B, Hk, L, D] bf16 GPU
    tensors of one shape and stride set, D a multiple of 16, 16-byte chunks."""
    return (isinstance(k_cache, torch.Tensor) and isinstance(v_cache, torch.Tensor)
            and k_cache.is_cuda and k_cache.dim() == 4 and k_cache.shape == v_cache.shape
            and k_cache.stride() == v_cache.stride() and k_cache.device == v_cache.device
            and k_cache.dtype == torch.bfloat16 and v_cache.dtype == torch.bfloat16
            and k_cache.shape[3] % 16 == 0 and _vec_ok(k_cache, v_cache))


def kv_inputs_ok(q, k, v, cos, sin, k_cache) -> bool:
    """Per-call inputs ``rope_kv_append`` takes for a cache that passed
    ``kv_cache_ok``: q [B,Hq,S,D], k and v [B,Hk,S,D] (HF's transposed
    views or contiguous), cos/sin [B or 1, S, D], all bf16 on the cache's
    device, 16-byte chunks."""
    bf = torch.bfloat16
    if not (q.dtype == bf and k.dtype == bf and v.dtype == bf and cos.dtype == bf
            and sin.dtype == bf):
        return False
    dev = k_cache.device
    if not (q.device == dev and k.device == dev and v.device == dev and cos.device == dev
            and sin.device == dev):
        return False
    if q.dim() != 4 or k.dim() != 4 or cos.dim() != 3:
        return False
    B, _, S, D = q.shape
    ks, cb, cs = k.shape, k_cache.shape, cos.shape
    return (ks[0] == B and ks[2] == S and ks[3] == D and v.shape == ks
            and cb[0] == B and cb[1] == ks[1] and cb[3] == D
            and cs == sin.shape and cs[1] == S and cs[2] == D and cs[0] in (1, B)
            and cos.stride() == sin.stride() and _vec_ok(q, k, v, cos, sin))


def kv_append_eligible(q, k, v, cos, sin, k_cache, v_cache) -> bool:
    """All of ``rope_kv_append``'s layout requirements (see the two checks)."""
    tensors = (q, k, v, cos, sin)
    return (all(isinstance(t, torch.Tensor) for t in tensors) and kv_cache_ok(k_cache, v_cache)
            and kv_inputs_ok(q, k, v, cos, sin, k_cache))


def kv_launch(q, k, v, cos, sin, k_cache, v_cache, pos: int,
              pos_t: torch.Tensor | None, norm=None) -> torch.Tensor:
    """Launch umic_rope_kv_append_bf16 (or, with ``norm = (q_w, k_w, eps)``,
    umic_qk_rmsnorm_rope_kv_append_bf16: q_norm / k_norm applied first) on
    inputs already checked by ``kv_append_eligible`` (and ``norm_weights_ok``);
    returns rope(q).  The C entry point re-validates strides, alignment and
    (without pos_t) the write range before launching."""
    B, Hq, S, D = q.shape
    q_out = torch.empty_like(q)
    qs, ks, vs, os_, cst = q.stride(), k.stride(), v.stride(), q_out.stride(), k_cache.stride()
    head = (q.data_ptr(), k.data_ptr(), v.data_ptr(), q_out.data_ptr(), k_cache.data_ptr(),
            v_cache.data_ptr(), cos.data_ptr(), sin.data_ptr())
    if norm is not None:
        name, head = ("umic_qk_rmsnorm_rope_kv_append_bf16",
                      head + (norm[0].data_ptr(), norm[1].data_ptr(), float(norm[2])))
    else:
        name = "umic_rope_kv_append_bf16"
    with _lib.device_of(q):
        _lib.call(name, *head, B, S, Hq, k.shape[1], D,
                  qs[0], qs[2], qs[1], ks[0], ks[2], ks[1], vs[0], vs[2], vs[1],
                  os_[0], os_[2], os_[1], cst[0], cst[1], cst[2], k_cache.shape[2], pos,
                  None if pos_t is None else pos_t.data_ptr(),
                  cos.stride(0) if cos.shape[0] == B else 0, cos.stride(1),
                  _lib.stream_of(q))
    return q_out


def norm_weights_ok(q, q_w, k_w) -> bool:
    """Head-row RMSNorm weights the fused norm + RoPE kernels take: [D] bf16,
    contiguous, 16-byte aligned, on q's device, with D = 128 or 256 -- the head
    sizes whose eager q_norm / k_norm reduction order the kernels reproduce
    (other sizes run the module norms, then the fused RoPE)."""
    D = q.shape[-1]
    if D not in (128, 256):
        return False
    return all(isinstance(w, torch.Tensor) and w.dtype == torch.bfloat16 and w.dim() == 1
               and w.shape[0] == D and w.is_contiguous() and w.device == q.device
               and w.data_ptr() % 16 == 0 for w in (q_w, k_w))


def qk_norm_rope_eligible(q, k, cos, sin, q_w, k_w) -> bool:
    """The HF text layout of ``text_rope_eligible`` with 16-byte chunks
    everywhere, plus norm weights the fused kernel takes."""
    return (text_rope_eligible(q, k, cos, sin) and norm_weights_ok(q, q_w, k_w)
            and _vec_ok(q, k, cos, sin))


def qk_norm_rope(q, k, cos, sin, q_w, k_w, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """The text attention's q_norm / k_norm on every head row, then HF
    apply_rotary_pos_emb, in one launch (umic_qk_rmsnorm_rope_bf16).

    q [B,Hq,S,D] and k [B,Hk,S,D] are the projections as HF views them
    (``proj(x).view(B,S,H,D).transpose(1,2)``) BEFORE the norms -- a head-row
    norm commutes with that transpose; q_w, k_w are the norms' [D] weights.
    Returns (q_embed, k_embed) allocated like eager's (``torch.empty_like``).
    Bit-identical to rmsnorm_hip on each head row followed by the text RoPE.
    """
    require_device(q, k, cos, sin, q_w, k_w)
    if not qk_norm_rope_eligible(q, k, cos, sin, q_w, k_w):
        raise ValueError(f"qk_norm_rope: unsupported layout q{tuple(q.shape)} k{tuple(k.shape)}")
    B, Hq, S, D = q.shape
    Hk = k.shape[1]
    q_out, k_out = torch.empty_like(q), torch.empty_like(k)
    qs, ks = _strides_bsh(q, "bhsd"), _strides_bsh(k, "bhsd")
    qos, kos = _strides_bsh(q_out, "bhsd"), _strides_bsh(k_out, "bhsd")
    with _lib.device_of(q):
        _lib.call("umic_qk_rmsnorm_rope_bf16", q.data_ptr(), k.data_ptr(), q_out.data_ptr(),
                  k_out.data_ptr(), q_w.data_ptr(), k_w.data_ptr(), float(eps),
                  cos.data_ptr(), sin.data_ptr(), B, S, Hq, Hk, D, *qs, *ks, *qos, *kos,
                  cos.stride(0) if cos.shape[0] == B else 0, cos.stride(1), _lib.stream_of(q))
    return q_out, k_out


def rope_kv_append(q, k, v, cos, sin, k_cache, v_cache, pos: int,
                   pos_t: torch.Tensor | None = None) -> torch.Tensor:
    """HF text RoPE of q and k fused with the append into an in-place cache.

    q [B,Hq,S,D], k/v [B,Hk,S,D] (HF's transposed views), cos/sin [B or 1,S,D]
    bf16; k_cache/v_cache [B,Hk,L,D].  Writes rope(k) and v at cache positions
    [P, P+S), P = pos (+ pos_t[0], an int64 device scalar, when given: the
    replay-safe form for captured graphs), and returns rope(q) allocated like
    eager's ``torch.empty_like(q)``.  One launch replaces the reference's
    make_text_rope (src/umic/kernels/rope.py:86-107) plus the cache append of
    src/umic/cache.py:59-70.  Without pos_t a write past the cache raises,
    as the reference does (src/umic/cache.py:65-68).
    """
    require_device(q, k, v, cos, sin, k_cache, v_cache)
    if not kv_append_eligible(q, k, v, cos, sin, k_cache, v_cache):
        raise ValueError("rope_kv_append: unsupported layout "
                         f"q{tuple(q.shape)} k{tuple(k.shape)} cache{tuple(k_cache.shape)}")
    S, L = q.shape[2], k_cache.shape[2]
    if pos_t is None and not (0 <= pos and pos + S <= L):
        raise RuntimeError(f"InplaceLayer overflow: pos {pos} + new {S} > buffer {L}")
    if pos_t is not None and not (pos_t.is_cuda and pos_t.dtype == torch.int64
                                  and pos_t.device == q.device and pos_t.numel() >= 1):
        raise ValueError("rope_kv_append: pos_t must be an int64 tensor on q's device")
    return kv_launch(q, k, v, cos, sin, k_cache, v_cache, pos, pos_t)


# Name of the reference's vision wrapper (src/umic/kernels/rope.py:78).
apply_rotary_vision_triton = apply_rotary_vision_hip
