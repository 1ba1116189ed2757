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


@pytest.mark.parametrize("Hq,Hk", [(8, 2), (8, 4), (6, 3)])
def test_text_rope_contiguous_and_batched(Hq, Hk):
    """Contiguous [B, H, S, D] q/k (head strides S * D) with two head rows
    per thread (8 / 2), four (8 / 4) and one (6 / 3), per-batch and
    batch-broadcast tables."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(1)
    B, S, D = 2, 100, 128
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


@pytest.mark.parametrize("S,Hq,Hk,D", [(300, 8, 2, 128), (20, 2, 1, 1024)])
def test_text_rope_unaligned_tables_take_the_staged_path(S, Hq, Hk, D):
    """bf16 tables are read per item with 16-byte loads when their bases and
    row strides allow it; tables at an odd element offset (2-byte aligned
    rows) or 4 elements in (8-byte aligned: staged with 8-byte moves) are
    staged through LDS instead -- by the lane-per-chunk kernel when a head
    row fits a wavefront (D = 128), else by the item-pair kernel (D = 1024).
    Same results every way."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(2)
    cos, sin = text_tables(S, D, 1e6)
    q = bf16_randn(1, S, Hq, D, gen=g).to(DEV).transpose(1, 2)
    k = bf16_randn(1, S, Hk, D, gen=g).to(DEV).transpose(1, 2)
    for shift in (0, 1, 4):
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


@pytest.mark.parametrize("S,H,D", [(300, 4, 128), (77, 6, 128), (19, 3, 256), (1, 4, 256)])
def test_vision_rope_bf16_tables_head_groups(S, H, D):
    """bf16 tables and head dims that are whole 128-byte half rows take the
    head-group kernel in its vision arithmetic (fp32 ops, one rounding): four
    (H = 4), two (6) or one (3) head rows per thread.  Bit for bit with the
    oracle on the exactly widened tables and with HF on the GPU."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb_vision

    print(f"vision head groups S={S} H={H} D={D}", flush=True)
    g = torch.Generator().manual_seed(S * 7 + D + H)
    qkv = bf16_randn(S, 3, H, D, gen=g)
    ang = 3.0 * torch.randn(S, D, generator=g)
    c, s_ = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    q, k, _ = qkv.to(DEV).permute(1, 0, 2, 3).unbind(0)
    qo, ko = rope.apply_rotary_vision_hip(q, k, c.to(DEV), s_.to(DEV))
    torch.cuda.synchronize()
    qc, kc, _ = qkv.permute(1, 0, 2, 3).unbind(0)
    cn, sn = c.float().numpy(), s_.float().numpy()
    assert np.array_equal(bits(qo), oracle.rope_vision(bits(qc), cn, sn))
    assert np.array_equal(bits(ko), oracle.rope_vision(bits(kc), cn, sn))
    rq, rk = apply_rotary_pos_emb_vision(q, k, c.to(DEV), s_.to(DEV))
    assert torch.equal(qo, rq) and torch.equal(ko, rk)


@pytest.mark.parametrize("S,H,D,cs_pad", [(37, 3, 16, 0), (50, 5, 32, 0), (19, 4, 48, 1),
                                          (64, 2, 96, 0), (23, 7, 112, 1), (11, 2, 256, 0),
                                          (9, 3, 512, 0), (300, 16, 80, 1), (1, 1, 80, 0)])
def test_vision_rope_lane_form_vs_oracle(S, H, D, cs_pad):
    """Head rows that fit a wavefront (D / 8 <= 64 chunks) take the
    lane-per-chunk kernel: 60 or 64 lanes per wavefront hold whole rows, the
    rotation partner D / 16 lanes away is fetched across lanes.  fp32 table
    rows 16-byte aligned (vector staging) or D + 1 floats apart (cs_pad:
    scalar staging).  Bit for bit with the oracle and with HF on the GPU."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb_vision

    print(f"vision lane form S={S} H={H} D={D} cs_pad={cs_pad}", flush=True)
    g = torch.Generator().manual_seed(S * 31 + D)
    qkv = bf16_randn(S, 3, H, D, gen=g)
    ang = 3.0 * torch.randn(S, D, generator=g)
    cbig = torch.zeros(S, D + cs_pad)
    sbig = torch.zeros(S, D + cs_pad)
    cbig[:, :D], sbig[:, :D] = ang.cos(), ang.sin()
    c, s_ = cbig.to(DEV)[:, :D], sbig.to(DEV)[:, :D]
    q, k, _ = qkv.to(DEV).permute(1, 0, 2, 3).unbind(0)
    qo, ko = rope.apply_rotary_vision_hip(q, k, c, s_)
    torch.cuda.synchronize()
    qc, kc, _ = qkv.permute(1, 0, 2, 3).unbind(0)
    cn, sn = cbig[:, :D].contiguous().numpy(), sbig[:, :D].contiguous().numpy()
    assert np.array_equal(bits(qo), oracle.rope_vision(bits(qc), cn, sn))
    assert np.array_equal(bits(ko), oracle.rope_vision(bits(kc), cn, sn))
    rq, rk = apply_rotary_pos_emb_vision(q, k, c, s_)
    assert torch.equal(qo, rq) and torch.equal(ko, rk)


def test_text_rope_lane_form_batched_staged_tables():
    """Batched text RoPE whose bf16 tables are staged (odd element offset)
    through the lane-per-chunk kernel, with a per-batch and a broadcast
    table: positions of both batches inside one block's table rows."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(3)
    B, S, Hq, Hk, D = 2, 7, 3, 1, 64
    cos, sin = text_tables(S, D, 1e6, B=B, offsets=(0, 40))
    q = bf16_randn(B, S, Hq, D, gen=g).to(DEV).transpose(1, 2)
    k = bf16_randn(B, S, Hk, D, gen=g).to(DEV).transpose(1, 2)
    for bsel in (slice(0, 2), slice(0, 1)):
        cb, sb = cos[bsel], sin[bsel]
        cbig = torch.zeros(cb.shape[0], S, D + 1, dtype=torch.bfloat16, device=DEV)
        sbig = torch.zeros_like(cbig)
        cbig[..., 1:] = cb.to(DEV)
        sbig[..., 1:] = sb.to(DEV)
        qo, ko = rope.apply_rotary_text_hip(q, k, cbig[..., 1:], sbig[..., 1:])
        rq, rk = apply_rotary_pos_emb(q, k, cb.to(DEV), sb.to(DEV))
        assert torch.equal(qo, rq) and torch.equal(ko, rk), bsel
