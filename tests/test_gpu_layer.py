"""GPU: a full Qwen3-VL decoder layer and a small ViT through umic.apply-style
injection (hidden 4096, 32 q / 8 kv heads, head_dim 128,
intermediate 12288, random N(0, 0.02) weights, norms 1 + N(0, 0.1)).

Prefill (M=3100) takes every fused kernel whose site wins there (P5, the
tiled down_proj, norms, RoPE; q/o_proj stay on hipBLASLt) -- checked by
counting the C-ABI calls -- and decode (M=1) takes the library's GEMV for the
GEMM sites while norms and RoPE stay fused.  Outputs are compared with the
unpatched layer on the same GPU within the GEMM tolerance.
"""

from __future__ import annotations

import collections

import pytest
import torch
from helpers import max_rel_err, qwen3_decoder_layer, rel_err

from umic import _lib, integrate

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::FutureWarning")]
DEV = "cuda"
TOL = 2e-2


@pytest.fixture
def call_log(monkeypatch):
    log = collections.Counter()
    real = _lib.call

    def spy(name, *args):
        log[name] += 1
        return real(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    yield log
    integrate.unfuse_rope()


def decoder_layer():
    return qwen3_decoder_layer(DEV)


@pytest.mark.parametrize("M", [3100, 1])
def test_decoder_layer_prefill_and_decode(M, call_log):
    layer, rot = decoder_layer()
    torch.manual_seed(1)
    h = torch.randn(1, M, 4096).to(torch.bfloat16).to(DEV)
    pos = torch.arange(M, device=DEV)[None]
    cos_sin = rot(h, pos)
    with torch.no_grad():
        ref = layer(h, position_embeddings=cos_sin)
        assert integrate.fuse_mlps(layer) == 1
        assert integrate.fuse_linears(layer) == 2
        assert integrate.fuse_rmsnorms(layer) == 4
        assert integrate.fuse_add_rmsnorm(layer) == 1
        assert integrate.fuse_text_rope()
        out = layer(h, position_embeddings=cos_sin)
        torch.cuda.synchronize()
    e1, e2 = max_rel_err(out, ref), rel_err(out, ref)
    print(f"decoder layer M={M}: max_rel {e1:.2e} rel {e2:.2e} calls {dict(call_log)}",
          flush=True)
    assert e1 <= TOL and e2 <= TOL
    assert call_log["umic_rmsnorm_bf16"] == 3          # input_layernorm, q_norm, k_norm
    assert call_log["umic_rope_qk_bf16"] == 1          # q and k in one launch
    if M == 1:
        # the post-attention residual add + RMSNorm folded into the P5 GEMV
        assert call_log["umic_add_rmsnorm_gate_silu_mul_bf16"] == 1
        assert call_log["umic_add_rmsnorm_bf16"] == 0
        assert call_log["umic_gate_silu_mul_bf16"] == 0
    else:
        # P5 on the tiled kernel after the fused add + RMSNorm
        assert call_log["umic_add_rmsnorm_bf16"] == 1
        assert call_log["umic_gate_silu_mul_bf16"] == 1
    if M == 1:
        # q_proj and o_proj on the GEMV; the down projection carries the MLP
        # residual add in its epilogue
        assert call_log["umic_linear_add_bf16"] == 1
        assert call_log["umic_linear_ws_bf16"] + call_log["umic_linear_bf16"] == 2
    else:
        # the MLP's down_proj on the tiled linear (in its row band); q/o_proj
        # stay on hipBLASLt, which the tiled linear only ties at this shape
        assert integrate.TILED_MIN_ROWS_DOWN <= M <= integrate.TILED_MAX_ROWS_DOWN
        assert integrate.TILED_MIN_ROWS_LINEAR is None
        assert call_log["umic_linear_add_bf16"] == 0
        assert call_log["umic_linear_ws_bf16"] == 1 and call_log["umic_linear_bf16"] == 0


def test_decoder_layer_prefill_with_tiled_qo(call_log, monkeypatch):
    """Prefill with the reference's own q/o rule (the tiled kernel from 64
    rows, src/umic/integrate.py:91,98-131): q_proj and o_proj
    then run on this library's tiled linear beside down_proj, and the layer
    still matches the unpatched one within the GEMM tolerance."""
    monkeypatch.setattr(integrate, "TILED_MIN_ROWS_LINEAR", 64)
    M = 3100
    layer, rot = decoder_layer()
    torch.manual_seed(1)
    h = torch.randn(1, M, 4096).to(torch.bfloat16).to(DEV)
    pos = torch.arange(M, device=DEV)[None]
    cos_sin = rot(h, pos)
    with torch.no_grad():
        ref = layer(h, position_embeddings=cos_sin)
        assert integrate.fuse_mlps(layer) == 1
        assert integrate.fuse_linears(layer) == 2
        assert integrate.fuse_rmsnorms(layer) == 4
        assert integrate.fuse_add_rmsnorm(layer) == 1
        assert integrate.fuse_text_rope()
        out = layer(h, position_embeddings=cos_sin)
        torch.cuda.synchronize()
    e1, e2 = max_rel_err(out, ref), rel_err(out, ref)
    print(f"decoder layer M={M}, tiled q/o: max_rel {e1:.2e} rel {e2:.2e} calls "
          f"{dict(call_log)}", flush=True)
    assert e1 <= TOL and e2 <= TOL
    # q_proj, o_proj and down_proj on the tiled linear
    assert call_log["umic_linear_ws_bf16"] + call_log["umic_linear_bf16"] == 3
    assert call_log["umic_gate_silu_mul_bf16"] == 1


def test_decoder_layer_with_autograd_runs_eager(call_log):
    """Grad mode on and weights requiring grad: the patched layer makes no
    kernel call (the kernels have no backward) and equals the unpatched layer
    bit for bit.  Only the forward runs here; SDPA is held to its flash and
    memory-efficient kernels."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    layer, rot = decoder_layer()
    torch.manual_seed(2)
    h = torch.randn(1, 256, 4096).to(torch.bfloat16).to(DEV)
    pos = torch.arange(256, device=DEV)[None]
    with torch.no_grad():
        cos_sin = rot(h, pos)
    assert layer.mlp.gate_proj.weight.requires_grad
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        ref = layer(h, position_embeddings=cos_sin)
        integrate.fuse_mlps(layer)
        integrate.fuse_linears(layer)
        integrate.fuse_rmsnorms(layer)
        integrate.fuse_add_rmsnorm(layer)
        assert integrate.fuse_text_rope()
        out = layer(h, position_embeddings=cos_sin)
        torch.cuda.synchronize()
        assert out.requires_grad and torch.equal(out, ref)
        assert sum(call_log.values()) == 0, dict(call_log)
        with torch.no_grad():
            layer(h, position_embeddings=cos_sin)
        torch.cuda.synchronize()
    assert call_log["umic_gate_silu_mul_bf16"] == 1 and call_log["umic_rope_qk_bf16"] == 1


def test_config1_mlp_block(call_log):
    """BASELINE config 1 on the GPU: x[256,1024] ~N(0,1) -> RMSNorm (eps 1e-6,
    weight 1+N(0,0.1)) -> gate/up 1024->3072 (no bias, N(0,0.02)) ->
    SiLU(gate)*up -> down 3072->1024, built from transformers' Qwen3-VL text
    modules and seeded in that order.  Fused against the unpatched block, the
    fused gate_silu_mul against the oracle (one rounding of the fp32 product),
    and every fused site counted."""
    import numpy as np
    from helpers import bits, ulp
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import (Qwen3VLTextMLP,
                                                                Qwen3VLTextRMSNorm)

    import oracle

    cfg = Qwen3VLTextConfig(hidden_size=1024, intermediate_size=3072, rms_norm_eps=1e-6)
    norm, mlp = Qwen3VLTextRMSNorm(1024, eps=1e-6), Qwen3VLTextMLP(cfg)
    torch.manual_seed(0)
    x = torch.randn(256, 1024)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(1024))
        for lin in (mlp.gate_proj, mlp.up_proj, mlp.down_proj):
            lin.weight.normal_(0, 0.02)
    block = torch.nn.Sequential(norm, mlp).to(torch.bfloat16).to(DEV).eval()
    x = x.to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        ref = block(x)
        assert integrate.fuse_rmsnorms(block) == 1 and integrate.fuse_mlps(block) == 1
        out = block(x)
        h = norm(x)
        from umic.kernels import fused_ffn
        p5 = fused_ffn.gate_silu_mul_hip(h, mlp.gate_proj.weight.t(), mlp.up_proj.weight.t())
        torch.cuda.synchronize()
    assert max_rel_err(out, ref) <= TOL and rel_err(out, ref) <= TOL, (max_rel_err(out, ref),
                                                                     rel_err(out, ref))
    want = oracle.gate_silu_mul(bits(h), bits(mlp.gate_proj.weight), bits(mlp.up_proj.weight))
    d = ulp(bits(p5), want)
    assert (d <= 1).mean() > 0.999, np.bincount(d.ravel())[:8]
    assert call_log["umic_rmsnorm_bf16"] == 2             # the block's norm, then h
    assert call_log["umic_gate_silu_mul_bf16"] == 2       # the block's MLP, then p5


@pytest.mark.parametrize("fp32_rotary", [False, True])
def test_vision_pipeline_on_gpu(call_log, fp32_rotary):
    """The vision encoder with every vision fusion injected.  With the whole
    model cast to bf16 the rotary tables are bf16; a bf16 checkpoint keeps
    the rotary inv_freq buffer fp32 (fp32_rotary), and cos/sin arrive fp32."""
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLVisionConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLVisionModel

    cfg = Qwen3VLVisionConfig(depth=4, hidden_size=1280, num_heads=16, intermediate_size=2560,
                              patch_size=16, temporal_patch_size=2, in_channels=3,
                              spatial_merge_size=2, out_hidden_size=2048,
                              num_position_embeddings=2304, deepstack_visual_indexes=[1],
                              attn_implementation="sdpa")
    torch.manual_seed(0)
    m = Qwen3VLVisionModel(cfg)
    inv_freq = m.rotary_pos_emb.inv_freq.clone()
    m = m.to(torch.bfloat16)
    if fp32_rotary:
        m.rotary_pos_emb.inv_freq = inv_freq
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, torch.nn.LayerNorm):
                mod.weight.add_(0.1 * torch.randn_like(mod.weight))
                mod.bias.add_(0.1 * torch.randn_like(mod.bias))
    m = m.to(DEV).eval()
    grid = torch.tensor([[1, 32, 32]] * 4, device=DEV)
    px = torch.randn(4 * 32 * 32, 3 * 2 * 16 * 16).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        ref = m(px, grid_thw=grid)
        integrate.fuse_layernorms(m)
        assert integrate.fuse_vision_rope()
        assert integrate.fuse_vision_encoder_pipeline(m) == 1
        assert integrate.fuse_gelu_mlps(m) == 4
        out = m(px, grid_thw=grid)
        torch.cuda.synchronize()
    for a, b in ((out.last_hidden_state, ref.last_hidden_state),
                 (out.pooler_output, ref.pooler_output),
                 (out.deepstack_features[0], ref.deepstack_features[0])):
        assert max_rel_err(a, b) <= TOL and rel_err(a, b) <= TOL, (max_rel_err(a, b),
                                                                   rel_err(a, b))
    # 4 blocks: norm1 of block 0 plain, 3 cross-block + 4 intra-block + merger
    # add+LN; the deepstack tap after block 1 keeps its plain add.
    assert call_log["umic_rope_qk_bf16"] == 4
    assert call_log["umic_add_layernorm_bf16"] == 4 + 2 + 1
    assert call_log["umic_layernorm_bf16"] == 2 + 1   # block 0 and 2 norm1, deepstack merger
    assert call_log["umic_linear_ws_bf16"] == 4       # each block's fc1 + tanh GELU


@pytest.mark.parametrize("act,rows", [("gelu_pytorch_tanh", 16384), ("gelu", 4100),
                                      ("gelu_pytorch_tanh", 63)])
def test_vit_gelu_mlp_module(act, rows, call_log):
    """The ViT MLP block at BASELINE's ViT width (hidden 1280, 4x MLP): fused
    fc1 + GELU then the vendor fc2, against the unpatched module; 63 rows stay
    on the eager path and match it bit for bit."""
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLVisionConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLVisionMLP

    cfg = Qwen3VLVisionConfig(hidden_size=1280, intermediate_size=5120, hidden_act=act)
    torch.manual_seed(5)
    mlp = Qwen3VLVisionMLP(cfg).to(torch.bfloat16).to(DEV).eval()
    with torch.no_grad():
        for lin in (mlp.linear_fc1, mlp.linear_fc2):
            lin.weight.normal_(0, 0.02)
            lin.bias.normal_(0, 0.1)
    x = torch.randn(rows, 1280, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        ref = mlp(x)
        assert integrate.fuse_gelu_mlps(mlp) == 1
        kind = mlp._umic_fc[2]
        out = mlp(x)
        torch.cuda.synchronize()
    assert kind == ("gelu_tanh" if act == "gelu_pytorch_tanh" else "gelu")
    if rows < integrate.FUSE_MIN_ROWS:
        assert call_log["umic_linear_ws_bf16"] == 0 and torch.equal(out, ref)
    else:
        assert call_log["umic_linear_ws_bf16"] == 1
        assert max_rel_err(out, ref) <= TOL and rel_err(out, ref) <= TOL, (max_rel_err(out, ref),
                                                                         rel_err(out, ref))
