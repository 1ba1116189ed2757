"""GPU parity: the text attention's per-head q_norm / k_norm fused with its
RoPE (``umic_qk_rmsnorm_rope_bf16``) and with RoPE plus the in-place KV
append (``umic_qk_rmsnorm_rope_kv_append_bf16``).

The oracle is the composition of two pinned oracle functions: ``rmsnorm`` on
every [D] head row, then ``rope_text`` -- the eager chain
``q_norm(q_proj(x).view(B,S,H,D))`` → ``apply_rotary_pos_emb``
(transformers modeling_qwen3_vl ``Qwen3VLTextAttention.forward``).  Checked
bit for bit at the BASELINE text shapes (config 5's 3094-token prefill, its
32-token flow step, a decode token), a batch of two with per-sequence
tables or one table broadcast over the batch, and both head sizes the
kernels take (D = 128: 8 lanes per head row, D = 256: 16 lanes), whose eager
reduction order they reproduce; other head sizes are rejected (the host then
runs the module norms).  Against the transformers modules on the GPU the
outputs are identical.  Weights are random, not ones, so a dropped or
swapped q/k weight fails.
"""

from __future__ import annotations

import collections

import numpy as np
import pytest
import torch
from helpers import (bf16_randn, bits, from_bits, log_parity, max_rel_err, qwen3_decoder_layer,
                     rel_err, ulp, ulp_hist)

import oracle
from umic import _lib, integrate
from umic.kernels import rope

from test_gpu_kv_cache import check, inputs, tables

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::FutureWarning")]
DEV = "cuda"
EPS = 1e-6

SHAPES = [
    (1, 3094, 32, 8, 128),     # config 5 prefill
    (1, 32, 32, 8, 128),       # flow step
    (1, 1, 32, 8, 128),        # decode token
    (2, 5, 4, 2, 128),         # batch of two, per-sequence tables
    (1, 9, 3, 1, 128),         # a ragged last block
    (1, 5, 2, 1, 256),         # 16 lanes per head row: the full-row DPP mirror
    (1, 300, 16, 4, 256),      # D = 256 at many rows
    (3, 7, 12, 4, 128),        # four rows per thread, batch of three, ragged last block
]


def weights(D, seed):
    g = torch.Generator().manual_seed(seed)
    return bf16_randn(D, scale=0.5, shift=1.0, gen=g), bf16_randn(D, scale=0.5, shift=1.0, gen=g)


def normed(x, w):
    """Oracle q_norm / k_norm of [..., D] bf16 head rows (a tensor)."""
    return from_bits(oracle.rmsnorm(bits(x), bits(w), EPS))


@pytest.mark.parametrize("B,S,Hq,Hk,D", SHAPES)
def test_qk_norm_rope_vs_oracle(B, S, Hq, Hk, D):
    print(f"qk_norm_rope B={B} S={S} Hq={Hq} Hk={Hk} D={D}", flush=True)
    qs, ks, _, _, _ = inputs(B, S, Hq, Hk, D, 1, seed=S + D)
    qw, kw = weights(D, seed=D)
    cos, sin = tables(B, S, D, 3000 if S < 64 else 0)
    q, k = (t.to(DEV).transpose(1, 2) for t in (qs, ks))
    qo, ko = rope.qk_norm_rope(q, k, cos.to(DEV), sin.to(DEV), qw.to(DEV), kw.to(DEV), EPS)
    torch.cuda.synchronize()
    assert qo.stride() == torch.empty_like(q).stride() and ko.shape == k.shape
    qn, kn = bits(normed(qs, qw)), bits(normed(ks, kw))
    for b in range(B):
        c, s = bits(cos)[b], bits(sin)[b]
        assert np.array_equal(bits(qo.transpose(1, 2))[b], oracle.rope_text(qn[b], c, s)), b
        assert np.array_equal(bits(ko.transpose(1, 2))[b], oracle.rope_text(kn[b], c, s)), b


def test_qk_norm_rope_broadcast_tables():
    """B = 2 against one [1, S, D] table broadcast over the batch (HF passes
    such tables when every sequence shares its positions)."""
    B, S, Hq, Hk, D = 2, 40, 4, 2, 128
    qs, ks, _, _, _ = inputs(B, S, Hq, Hk, D, 1, seed=31)
    qw, kw = weights(D, seed=32)
    cos, sin = tables(1, S, D, 17)
    q, k = (t.to(DEV).transpose(1, 2) for t in (qs, ks))
    assert rope.qk_norm_rope_eligible(q, k, cos.to(DEV), sin.to(DEV), qw.to(DEV), kw.to(DEV))
    qo, ko = rope.qk_norm_rope(q, k, cos.to(DEV), sin.to(DEV), qw.to(DEV), kw.to(DEV), EPS)
    torch.cuda.synchronize()
    qn, kn = bits(normed(qs, qw)), bits(normed(ks, kw))
    c, s = bits(cos)[0], bits(sin)[0]
    for b in range(B):
        assert np.array_equal(bits(qo.transpose(1, 2))[b], oracle.rope_text(qn[b], c, s)), b
        assert np.array_equal(bits(ko.transpose(1, 2))[b], oracle.rope_text(kn[b], c, s)), b


@pytest.mark.parametrize("D", [64, 512, 1024])
def test_qk_norm_rope_rejects_other_head_sizes(D):
    """Head sizes whose eager q_norm / k_norm order the kernels do not
    reproduce are refused before any launch (the host then runs the module
    norms), and the Python gate says so."""
    qs, ks, vs, kc, vc = inputs(1, 4, 2, 1, D, 8, seed=D)
    qw, kw = (w.to(DEV) for w in weights(D, seed=D))
    q, k, v = (t.to(DEV).transpose(1, 2) for t in (qs, ks, vs))
    assert not rope.norm_weights_ok(q, qw, kw)
    cos, sin = (t.to(DEV) for t in tables(1, 4, D, 0))
    qo, ko = torch.empty_like(q), torch.empty_like(k)

    def bsh(t):  # (batch, position, head) strides of a [B, H, S, D] view
        return t.stride(0), t.stride(2), t.stride(1)

    rc = _lib.lib().umic_qk_rmsnorm_rope_bf16(
        q.data_ptr(), k.data_ptr(), qo.data_ptr(), ko.data_ptr(), qw.data_ptr(), kw.data_ptr(),
        EPS, cos.data_ptr(), sin.data_ptr(), 1, 4, 2, 1, D, *bsh(q), *bsh(k), *bsh(qo),
        *bsh(ko), cos.stride(0), cos.stride(1), _lib.stream_of(q))
    torch.cuda.synchronize()
    assert rc == _lib.UMIC_ERR_UNSUPPORTED


@pytest.mark.parametrize("S", [3100, 32, 1])
def test_qk_norm_rope_vs_transformers(S):
    """Against the modules themselves on the GPU: Qwen3VLTextRMSNorm on the
    [1, S, H, 128] q and k projections, then apply_rotary_pos_emb -- at the
    BASELINE prefill (q_norm over 99200 rows, k_norm over 24800), a flow step
    and a decode token.  Within one bf16 ulp (the bar), and identical."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import (Qwen3VLTextRMSNorm,
                                                                apply_rotary_pos_emb)

    B, Hq, Hk, D = 1, 32, 8, 128
    qs, ks, _, _, _ = inputs(B, S, Hq, Hk, D, 1, seed=11)
    qw, kw = weights(D, seed=12)
    cos, sin = (t.to(DEV) for t in tables(B, S, D, 0))
    qn_mod = Qwen3VLTextRMSNorm(D, eps=EPS).to(DEV, torch.bfloat16)
    kn_mod = Qwen3VLTextRMSNorm(D, eps=EPS).to(DEV, torch.bfloat16)
    with torch.no_grad():
        qn_mod.weight.copy_(qw)
        kn_mod.weight.copy_(kw)
        qr, kr = apply_rotary_pos_emb(qn_mod(qs.to(DEV)).transpose(1, 2),
                                      kn_mod(ks.to(DEV)).transpose(1, 2), cos, sin)
        qo, ko = rope.qk_norm_rope(qs.to(DEV).transpose(1, 2), ks.to(DEV).transpose(1, 2),
                                   cos, sin, qw.to(DEV), kw.to(DEV), EPS)
    torch.cuda.synchronize()
    for name, got, ref, H in (("q", qo, qr, Hq), ("k", ko, kr, Hk)):
        d = ulp(bits(got), bits(ref))
        log_parity(f"qk_norm_rope ({name})", (B, H, S, D), d)
        assert d.max() <= 1, ulp_hist(d)
        assert (d == 0).all(), ulp_hist(d)


@pytest.mark.parametrize("B,S,Hq,Hk,D,pos,L", [
    (1, 3094, 32, 8, 128, 0, 3200),      # prefill into a fresh cache
    (1, 32, 32, 8, 128, 3094, 3200),     # flow step after the prefix
    (1, 1, 32, 8, 128, 3126, 3200),      # decode token
    (2, 5, 4, 2, 128, 7, 16),            # batch of two
    (1, 9, 3, 1, 128, 0, 9),             # exactly fills the cache
    (1, 6, 2, 1, 256, 3, 12),            # 16 lanes per head row
])
def test_qk_norm_rope_kv_append_vs_oracle(B, S, Hq, Hk, D, pos, L):
    print(f"qk_norm_rope_kv_append B={B} S={S} Hq={Hq} Hk={Hk} D={D} pos={pos} L={L}",
          flush=True)
    qs, ks, vs, kc0, vc0 = inputs(B, S, Hq, Hk, D, L, seed=S + D + 1)
    qw, kw = weights(D, seed=D + 1)
    cos, sin = tables(B, S, D, pos)
    q, k, v = (t.to(DEV).transpose(1, 2) for t in (qs, ks, vs))
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    cos_d, sin_d, qw_d, kw_d = cos.to(DEV), sin.to(DEV), qw.to(DEV), kw.to(DEV)
    assert rope.kv_append_eligible(q, k, v, cos_d, sin_d, kc, vc)
    assert rope.norm_weights_ok(q, qw_d, kw_d)
    qo = rope.kv_launch(q, k, v, cos_d, sin_d, kc, vc, pos, None, (qw_d, kw_d, EPS))
    torch.cuda.synchronize()
    check(qo, kc, vc, normed(qs, qw), normed(ks, kw), vs, kc0, vc0, cos, sin,
          list(range(pos, pos + S)))


def test_qk_norm_rope_kv_append_device_position():
    """Graph-mode form: rows written at the device position, rows outside
    the cache dropped, q still normed and rotated."""
    B, S, Hq, Hk, D, L = 1, 4, 2, 1, 128, 8
    qs, ks, vs, kc0, vc0 = inputs(B, S, Hq, Hk, D, L, seed=21)
    qw, kw = weights(D, seed=22)
    cos, sin = tables(B, S, D, 0)
    q, k, v = (t.to(DEV).transpose(1, 2) for t in (qs, ks, vs))
    for p, rows in ((6, [6, 7, None, None]), (-2, [None, None, 0, 1])):
        kc, vc = kc0.to(DEV), vc0.to(DEV)
        pos_t = torch.tensor([p], dtype=torch.int64, device=DEV)
        qo = rope.kv_launch(q, k, v, cos.to(DEV), sin.to(DEV), kc, vc, 0, pos_t,
                            (qw.to(DEV), kw.to(DEV), EPS))
        torch.cuda.synchronize()
        check(qo, kc, vc, normed(qs, qw), normed(ks, kw), vs, kc0, vc0, cos, sin, rows)


@pytest.fixture
def call_log(monkeypatch):
    log = collections.Counter()
    real = _lib.call

    def spy(name, *args):
        log[name] += 1
        return real(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    yield log


def test_decoder_layer_without_inplace_cache(call_log):
    """fuse_kv_rope on a BASELINE config 5 decoder layer with a
    DynamicCache: q_norm, k_norm and RoPE are one launch, the cache's own
    update follows.  The cached keys are the oracle's (from the layer's own
    k projection), the layer output within the GEMM tolerance of eager.
    Attention is held to the flash / memory-efficient SDPA kernels."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from transformers.cache_utils import DynamicCache

    layer, rot = qwen3_decoder_layer(DEV)
    attn = layer.self_attn
    S = 300
    torch.manual_seed(5)
    x = torch.randn(1, S, 4096).to(torch.bfloat16).to(DEV)
    cs = rot(x, torch.arange(S, device=DEV)[None])
    with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION,
                                       SDPBackend.EFFICIENT_ATTENTION]):
        dyn_ref, dyn = DynamicCache(), DynamicCache()
        ref = layer(x, position_embeddings=cs, past_key_values=dyn_ref)
        assert integrate.fuse_kv_rope(layer) == 1
        out = layer(x, position_embeddings=cs, past_key_values=dyn)
        k_raw = attn.k_proj(layer.input_layernorm(x)).view(1, S, -1, 128)
        torch.cuda.synchronize()
    assert call_log["umic_qk_rmsnorm_rope_bf16"] == 1
    kn = oracle.rmsnorm(bits(k_raw), bits(attn.k_norm.weight), attn.k_norm.variance_epsilon)
    krot = oracle.rope_text(kn[0], bits(cs[0])[0], bits(cs[1])[0])        # [S, Hk, D]
    assert np.array_equal(bits(dyn.layers[0].keys)[0], krot.transpose(1, 0, 2))
    assert torch.equal(dyn.layers[0].values, dyn_ref.layers[0].values)
    assert torch.equal(dyn.layers[0].keys, dyn_ref.layers[0].keys)
    e1, e2 = max_rel_err(out, ref), rel_err(out, ref)
    print(f"layer with fused q/k norm + rope: max_rel {e1:.2e} rel {e2:.2e}", flush=True)
    assert e1 <= 2e-2 and e2 <= 2e-2
