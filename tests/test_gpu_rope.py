"""GPU parity: fused q+k RoPE (text bf16-per-op mode, vision fp32 mode).

Inputs are laid out exactly as the transformers qwen3_vl attention hands them
over: text q/k are transposed [B,H,S,D] views of [B,S,H,D] projections with
cos/sin from the text rotary embedding (theta 1e6); vision q/k are strided
views of a packed [S,3,H,80] qkv with fp32 cos/sin from merged h/w grid ids
(theta 1e4).  Outputs are compared bit for bit with the CPU oracle and with
the eager transformers functions run on the same GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from helpers import bf16_randn, bits, log_parity, ulp

import oracle
from umic.kernels import rope

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::FutureWarning")]
DEV = "cuda"


def text_tables(S, D, theta, B=1, offsets=(0,)):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextRotaryEmbedding

    cfg = Qwen3VLTextConfig(hidden_size=8 * D, num_attention_heads=8, num_key_value_heads=8,
                            head_dim=D, rope_parameters={"rope_type": "default",
                                                         "rope_theta": theta})
    rot = Qwen3VLTextRotaryEmbedding(cfg)
    pos = torch.stack([torch.arange(o, o + S) for o in offsets])[:B]
    dummy = torch.zeros(1, dtype=torch.bfloat16)
    return rot(dummy, pos)  # bf16 [B, S, D]


def vision_tables(grid, D, merge=2):
    from transformers import vision_utils as vu
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLVisionRotaryEmbedding

    pid = vu.get_vision_position_ids(torch.tensor(grid), merge)
    emb = Qwen3VLVisionRotaryEmbedding(D // 2)(pid).reshape(pid.shape[0], -1)
    emb = torch.cat((emb, emb), -1)
    return emb.cos(), emb.sin()


@pytest.mark.parametrize("S,Hq,Hk,D", [(3100, 32, 8, 128), (37, 4, 2, 64), (1, 32, 8, 128),
                                       (5, 3, 1, 6), (9, 2, 2, 2), (7, 2, 1, 1024), (5, 2, 2, 4)])
def test_text_rope_hf_layout(S, Hq, Hk, D):
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(S + D)
    cos, sin = text_tables(S, D, 1e6, offsets=(S * 3,))
    qs = bf16_randn(1, S, Hq, D, gen=g)
    ks = bf16_randn(1, S, Hk, D, gen=g)
    q, k = qs.to(DEV).transpose(1, 2), ks.to(DEV).transpose(1, 2)
    qo, ko = rope.apply_rotary_text_hip(q, k, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    assert qo.shape == q.shape and qo.stride() == q.stride()
    assert np.array_equal(bits(qo.transpose(1, 2))[0], oracle.rope_text(bits(qs)[0], bits(cos)[0],
                                                                        bits(sin)[0]))
    assert np.array_equal(bits(ko.transpose(1, 2))[0], oracle.rope_text(bits(ks)[0], bits(cos)[0],
                                                                        bits(sin)[0]))
    rq, rk = apply_rotary_pos_emb(q, k, cos.to(DEV), sin.to(DEV))
    for name, got, ref in (("q", qo, rq), ("k", ko, rk)):
        d = ulp(bits(got), bits(ref))
        log_parity(f"text_rope ({name})", tuple(ref.shape), d)
        assert d.max() <= 1
    assert torch.equal(qo, rq) and torch.equal(ko, rk)


def test_text_rope_contiguous_and_batched():
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(1)
    B, S, Hq, Hk, D = 2, 100, 8, 2, 128
    cos, sin = text_tables(S, D, 1e6, B=B, offsets=(0, 500))
    q = bf16_randn(B, Hq, S, D, gen=g).to(DEV)          # contiguous [B,H,S,D]
    k = bf16_randn(B, Hk, S, D, gen=g).to(DEV)
    qo, ko = rope.apply_rotary_text_hip(q, k, cos.to(DEV), sin.to(DEV))
    rq, rk = apply_rotary_pos_emb(q, k, cos.to(DEV), sin.to(DEV))
    assert torch.equal(qo, rq) and torch.equal(ko, rk)
    # batch-broadcast table ([1, S, D] for B = 2)
    qo1, ko1 = rope.apply_rotary_text_hip(q, k, cos[:1].to(DEV), sin[:1].to(DEV))
    rq1, rk1 = apply_rotary_pos_emb(q, k, cos[:1].to(DEV), sin[:1].to(DEV))
    assert torch.equal(qo1, rq1) and torch.equal(ko1, rk1)


def test_text_rope_unaligned_tables_take_the_staged_path():
    """bf16 tables are read per item with 16-byte loads when their bases and
    row strides allow it; tables at an odd element offset (2-byte aligned
    rows) are staged through LDS instead -- same results either way."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(2)
    S, Hq, Hk, D = 300, 8, 2, 128
    cos, sin = text_tables(S, D, 1e6)
    q = bf16_randn(1, S, Hq, D, gen=g).to(DEV).transpose(1, 2)
    k = bf16_randn(1, S, Hk, D, gen=g).to(DEV).transpose(1, 2)
    for shift in (0, 1):
        cbig = torch.zeros(1, S, D + 8, dtype=torch.bfloat16, device=DEV)
        sbig = torch.zeros_like(cbig)
        cbig[..., shift:shift + D] = cos.to(DEV)
        sbig[..., shift:shift + D] = sin.to(DEV)
        c, s_ = cbig[..., shift:shift + D], sbig[..., shift:shift + D]
        assert (c.data_ptr() % 16 == 0) == (shift == 0)
        qo, ko = rope.apply_rotary_text_hip(q, k, c, s_)
        rq, rk = apply_rotary_pos_emb(q, k, cos.to(DEV), sin.to(DEV))
        assert torch.equal(qo, rq) and torch.equal(ko, rk), shift


@pytest.mark.parametrize("grid,H", [([[1, 32, 32]] * 16, 16), ([[1, 4, 6], [1, 6, 4]], 3),
                                    ([[2, 4, 4]], 1)])
def test_vision_rope_packed_qkv(grid, H):
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb_vision

    D = 80
    cos, sin = vision_tables(grid, D)
    S = cos.shape[0]
    g = torch.Generator().manual_seed(S)
    qkv = bf16_randn(S, 3, H, D, gen=g)
    q, k, _ = qkv.to(DEV).permute(1, 0, 2, 3).unbind(0)  # strided views
    qo, ko = rope.apply_rotary_vision_hip(q, k, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    assert qo.is_contiguous() and qo.shape == q.shape
    qc, kc, _ = qkv.permute(1, 0, 2, 3).unbind(0)
    assert np.array_equal(bits(qo), oracle.rope_vision(bits(qc), cos.numpy(), sin.numpy()))
    assert np.array_equal(bits(ko), oracle.rope_vision(bits(kc), cos.numpy(), sin.numpy()))
    rq, rk = apply_rotary_pos_emb_vision(q, k, cos.to(DEV), sin.to(DEV))
    for name, got, ref in (("q", qo, rq), ("k", ko, rk)):
        d = ulp(bits(got), bits(ref))
        log_parity(f"vision_rope ({name})", tuple(ref.shape), d)
        assert d.max() <= 1
    assert torch.equal(qo, rq) and torch.equal(ko, rk)


def test_vision_rope_bf16_tables_and_fallback_wrapper():
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb_vision

    cos, sin = vision_tables([[1, 8, 8]], 64)
    cos, sin = cos.to(torch.bfloat16).to(DEV), sin.to(torch.bfloat16).to(DEV)
    g = torch.Generator().manual_seed(2)
    q = bf16_randn(64, 4, 64, gen=g).to(DEV)
    k = bf16_randn(64, 2, 64, gen=g).to(DEV)
    fused = rope.make_vision_rope(apply_rotary_pos_emb_vision)
    qo, ko = fused(q, k, cos, sin)
    rq, rk = apply_rotary_pos_emb_vision(q, k, cos, sin)
    assert torch.equal(qo, rq) and torch.equal(ko, rk)
