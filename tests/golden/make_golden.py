"""Write tests/golden/umic_golden.npz: input/output vectors of the eager ops.

The reference (soonhong99/umic-alpamayo) ships no golden vectors; its only
numeric check is scripts/check_env.py:106-171 (seed 0, rel-err < 2e-2 vs
inline eager formulas).  The eager op chains its kernels replace live in the
third-party packages torch and transformers (qwen3_vl), so the fixtures are
those packages' own functions evaluated on the CPU here, in bf16, on seeded
inputs:

  rmsnorm        Qwen3VLTextRMSNorm.forward            (modeling_qwen3_vl.py:400-405)
  add_rmsnorm    residual + x, then the RMSNorm        (decoder layer, :559-563)
  layernorm      nn.LayerNorm (torch layer_norm)        (ViT norm1/norm2, :283-284)
  add_layernorm  h + x, then the LayerNorm             (ViT block, :299-305)
  rope_text      apply_rotary_pos_emb with cos/sin from Qwen3VLTextRotaryEmbedding
                 (theta 1e6, head_dim 128)              (:340-370, :412-435)
  rope_vision    apply_rotary_pos_emb_vision with cos/sin from the vision
                 rotary embedding over 2x2-merged h/w grid ids (theta 1e4)
                                                         (:110-119, :145-156, :706-713)
  mlp            Qwen3VLTextMLP front half silu(gate(x)) * up(x) and the
                 full MLP                                (:510-523)
  linear         nn.Linear (F.linear)

Every array is stored as uint16 bf16 bits (fp32 tables as float32).  Run:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "umic_golden.npz")


def bits(t: torch.Tensor) -> np.ndarray:
    assert t.dtype == torch.bfloat16
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main() -> None:
    from transformers.models.qwen3_vl import modeling_qwen3_vl as hf
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers import vision_utils as vu

    bf = torch.bfloat16
    torch.manual_seed(0)
    g: dict[str, np.ndarray] = {}

    # RMSNorm / add+RMSNorm, LM width slice
    M, N = 24, 1024
    x = torch.randn(M, N).to(bf)
    r = torch.randn(M, N).to(bf)
    w = (1 + 0.1 * torch.randn(N)).to(bf)
    norm = hf.Qwen3VLTextRMSNorm(N, eps=1e-6).to(bf)
    with torch.no_grad():
        norm.weight.copy_(w)
        g["rms_x"], g["rms_r"], g["rms_w"] = bits(x), bits(r), bits(w)
        g["rms_y"] = bits(norm(x))
        s = r + x
        g["addrms_s"], g["addrms_y"] = bits(s), bits(norm(s))

    # q_norm-shaped rows (head_dim 128)
    xq = torch.randn(64, 128).to(bf)
    wq = (1 + 0.1 * torch.randn(128)).to(bf)
    qn = hf.Qwen3VLTextRMSNorm(128, eps=1e-6).to(bf)
    with torch.no_grad():
        qn.weight.copy_(wq)
        g["rmsq_x"], g["rmsq_w"], g["rmsq_y"] = bits(xq), bits(wq), bits(qn(xq))

    # LayerNorm / add+LayerNorm, ViT width
    M, N = 32, 1280
    x = torch.randn(M, N).to(bf)
    r = torch.randn(M, N).to(bf)
    w = (1 + 0.1 * torch.randn(N)).to(bf)
    b = (0.1 * torch.randn(N)).to(bf)
    ln = torch.nn.LayerNorm(N, eps=1e-6).to(bf)
    with torch.no_grad():
        ln.weight.copy_(w)
        ln.bias.copy_(b)
        g["ln_x"], g["ln_r"], g["ln_w"], g["ln_b"] = bits(x), bits(r), bits(w), bits(b)
        g["ln_y"] = bits(ln(x))
        s = r + x
        g["addln_s"], g["addln_y"] = bits(s), bits(ln(s))

    # Text RoPE: q [1,4,S,128], k [1,2,S,128] as HF produces them (transposed
    # views of [1,S,H,D]), cos/sin from the text rotary embedding.
    S, Hq, Hk, D = 48, 4, 2, 128
    cfg = Qwen3VLTextConfig(hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hk,
                            head_dim=D, rope_parameters={"rope_type": "default",
                                                         "rope_theta": 1e6})
    rot = hf.Qwen3VLTextRotaryEmbedding(cfg)
    pos = torch.arange(1000, 1000 + S)[None, :]  # arbitrary offset: non-trivial angles
    q = torch.randn(1, S, Hq, D).to(bf).transpose(1, 2)
    k = torch.randn(1, S, Hk, D).to(bf).transpose(1, 2)
    cos, sin = rot(q, pos)
    assert cos.dtype == bf and cos.shape == (1, S, D)
    qe, ke = hf.apply_rotary_pos_emb(q, k, cos, sin)
    g["rt_q"], g["rt_k"] = bits(q.transpose(1, 2)), bits(k.transpose(1, 2))  # stored [1,S,H,D]
    g["rt_cos"], g["rt_sin"] = bits(cos), bits(sin)
    g["rt_qo"], g["rt_ko"] = bits(qe.transpose(1, 2)), bits(ke.transpose(1, 2))

    # Vision RoPE: 2 images of 4x6 patches, merge size 2, head_dim 80.
    grid = torch.tensor([[1, 4, 6], [1, 6, 4]])
    pid = vu.get_vision_position_ids(grid, 2)
    vrot = hf.Qwen3VLVisionRotaryEmbedding(80 // 2)
    emb = vrot(pid).reshape(pid.shape[0], -1)
    emb = torch.cat((emb, emb), dim=-1)
    vcos, vsin = emb.cos(), emb.sin()
    Sv, Hv = pid.shape[0], 3
    qkv = torch.randn(Sv, 3, Hv, 80).to(bf)
    vq, vk, _ = qkv.permute(1, 0, 2, 3).unbind(0)
    vqe, vke = hf.apply_rotary_pos_emb_vision(vq, vk, vcos, vsin)
    g["rv_q"], g["rv_k"] = bits(vq), bits(vk)
    g["rv_cos"], g["rv_sin"] = vcos.float().numpy(), vsin.float().numpy()
    g["rv_qo"], g["rv_ko"] = bits(vqe), bits(vke)

    # MLP (P5 motif) and linear, small width
    M, H, I = 32, 128, 256
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig as TC
    mcfg = TC(hidden_size=H, intermediate_size=I, hidden_act="silu")
    mlp = hf.Qwen3VLTextMLP(mcfg).to(bf)
    with torch.no_grad():
        for lin in (mlp.gate_proj, mlp.up_proj, mlp.down_proj):
            lin.weight.copy_((0.02 * torch.randn_like(lin.weight, dtype=torch.float32)).to(bf))
        x = torch.randn(M, H).to(bf)
        g["mlp_x"] = bits(x)
        g["mlp_wg"], g["mlp_wu"] = bits(mlp.gate_proj.weight), bits(mlp.up_proj.weight)
        g["mlp_wd"] = bits(mlp.down_proj.weight)
        g["mlp_h"] = bits(mlp.act_fn(mlp.gate_proj(x)) * mlp.up_proj(x))
        g["mlp_y"] = bits(mlp(x))
        lin = torch.nn.Linear(H, 192, bias=True).to(bf)
        lin.weight.copy_((0.02 * torch.randn(192, H)).to(bf))
        lin.bias.copy_((0.1 * torch.randn(192)).to(bf))
        g["lin_w"], g["lin_b"] = bits(lin.weight), bits(lin.bias)
        g["lin_y"] = bits(lin(x))

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(g)} arrays)")


if __name__ == "__main__":
    main()
