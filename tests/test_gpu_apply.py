"""GPU: ``umic.apply()`` end to end on a small random-weight Alpamayo-style
model (reference src/umic/optimize.py:92-168).

The wrapper holds ``vlm`` (a Qwen3-VL model: language model plus ViT) and
``expert`` (a Qwen3-VL text trunk that extends the VLM's KV cache with action
tokens and crops back, the flow loop's access pattern).  Everything is run
unpatched first; then ``umic.apply(model)`` with the default config patches
it in place and the same work runs again:

* greedy ``generate()`` of a text prompt and of an image + text prompt: the
  same tokens, per-step scores within the GEMM tolerance;
* the ViT alone on the same image: merged and deepstack features within the
  GEMM tolerance;
* three expert steps on a copy of the prompt's KV cache, each cropped back:
  bit-identical (norms, RoPE and the cache append are bit-exact; the expert
  keeps its vendor GEMMs).

The report's counts must equal the fuse functions' dry-run counts, and the
C-ABI call log must show every fused kernel family running: norms,
add+norms, text and vision RoPE (prefill, and the in-place append inside the
decode graphs), the tiled GEMMs at prefill and the GEMVs at decode.
Attention is held to the flash / memory-efficient SDPA kernels.
"""

from __future__ import annotations

import collections

import pytest
import torch
from helpers import max_rel_err

import umic
from umic import _lib, integrate

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::FutureWarning"),
              pytest.mark.filterwarnings("ignore::UserWarning")]
DEV = "cuda"
NEW = 8
TOL = 2e-2
IMG, VID, VSTART, VEND = 500, 501, 502, 503


def small_model():
    from torch import nn
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import (Qwen3VLForConditionalGeneration,
                                                                Qwen3VLTextModel)

    text = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=4, head_dim=128, vocab_size=512,
                rope_parameters={"rope_type": "default", "rope_theta": 1e6,
                                 "mrope_section": [24, 20, 20], "mrope_interleaved": True})
    cfg = Qwen3VLConfig(
        text_config=text,
        vision_config=dict(depth=2, hidden_size=128, num_heads=2, intermediate_size=256,
                           out_hidden_size=256, patch_size=8, temporal_patch_size=2,
                           spatial_merge_size=2, num_position_embeddings=64,
                           deepstack_visual_indexes=[0]),
        image_token_id=IMG, video_token_id=VID, vision_start_token_id=VSTART,
        vision_end_token_id=VEND)
    cfg._attn_implementation = "sdpa"
    cfg.text_config._attn_implementation = "sdpa"
    cfg.vision_config._attn_implementation = "sdpa"
    torch.manual_seed(0)
    vlm = Qwen3VLForConditionalGeneration(cfg)
    expert = Qwen3VLTextModel(cfg.text_config)
    for mod in (vlm, expert):
        with torch.no_grad():
            for name, p in mod.named_parameters():
                if "norm" in name:
                    p.copy_(1 + 0.1 * torch.randn_like(p))
                elif "bias" in name:
                    p.copy_(0.1 * torch.randn_like(p))
    root = nn.Module()
    root.vlm = vlm.to(torch.bfloat16).to(DEV).eval()
    root.expert = expert.to(torch.bfloat16).to(DEV).eval()
    return root


def generate(vlm, ids, **kw):
    out = vlm.generate(input_ids=ids, attention_mask=torch.ones_like(ids), max_new_tokens=NEW,
                       do_sample=False, output_scores=True, return_dict_in_generate=True, **kw)
    torch.cuda.synchronize()
    return out.sequences.cpu(), torch.stack(out.scores).float().cpu()


def copy_cache(cache):
    from transformers.cache_utils import DynamicCache

    c = DynamicCache()
    for i, lyr in enumerate(cache.layers):
        c.update(lyr.keys.clone(), lyr.values.clone(), i)
    return c


def expert_steps(expert, prefix, acts):
    """The flow loop's pattern: append the action tokens, read, crop back."""
    cache, n = copy_cache(prefix), prefix.get_seq_length()
    outs = []
    for a in acts:
        outs.append(expert(inputs_embeds=a, past_key_values=cache,
                           use_cache=True).last_hidden_state.clone())
        extra = cache.get_seq_length() - n
        if extra:
            cache.crop(-extra)
    torch.cuda.synchronize()
    return outs


def test_apply_end_to_end(monkeypatch):
    from torch.nn.attention import SDPBackend, sdpa_kernel

    model = small_model()
    vlm, expert = model.vlm, model.expert
    g = torch.Generator().manual_seed(1)
    text_ids = torch.randint(0, 500, (1, 80), generator=g).to(DEV)
    grid = torch.tensor([[1, 16, 16]], device=DEV)
    px = torch.randn(256, 3 * 2 * 8 * 8, generator=g).to(torch.bfloat16).to(DEV)
    img_ids = torch.cat([torch.randint(0, 500, (1, 6), generator=g),
                         torch.tensor([[VSTART] + [IMG] * 64 + [VEND]]),
                         torch.randint(0, 500, (1, 14), generator=g)], 1).to(DEV)
    acts = [torch.randn(1, 8, 256, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    attn = sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION])
    with torch.no_grad(), attn:
        ref_text = generate(vlm, text_ids)
        ref_img = generate(vlm, img_ids, pixel_values=px, image_grid_thw=grid)
        ref_vit = vlm.model.visual(px, grid_thw=grid)
        prefix = vlm.model.language_model(input_ids=text_ids, use_cache=True).past_key_values
        ref_exp = expert_steps(expert, prefix, acts)

        lm, visual = vlm.model.language_model, vlm.model.visual
        dry = {"lm_mlp_fused": integrate.fuse_mlps(lm, dry_run=True),
               "lm_rmsnorm_fused": integrate.fuse_rmsnorms(lm, dry_run=True),
               "lm_add_rmsnorm_fused": integrate.fuse_add_rmsnorm(lm, dry_run=True),
               "lm_kv_rope_fused": integrate.fuse_kv_rope(lm, dry_run=True),
               "ve_layernorm_fused": integrate.fuse_layernorms(visual, dry_run=True),
               "ve_pipeline_fused": integrate.fuse_vision_encoder_pipeline(visual, dry_run=True),
               "ve_gelu_mlp_fused": integrate.fuse_gelu_mlps(visual, dry_run=True),
               "expert_rmsnorm_fused": integrate.fuse_rmsnorms(expert, dry_run=True),
               "expert_add_rmsnorm_fused": integrate.fuse_add_rmsnorm(expert, dry_run=True),
               "expert_kv_rope_fused": integrate.fuse_kv_rope(expert, dry_run=True)}
        log = collections.Counter()
        real = _lib.call

        def spy(name, *args):
            log[name] += 1
            return real(name, *args)

        monkeypatch.setattr(_lib, "call", spy)
        try:
            report = umic.apply(model)
            print("report", report, flush=True)
            for key, n in dry.items():
                assert n > 0 and report[key] == n, (key, report.get(key), n)
            assert report["lm_linear_fused"] == 4
            assert report["text_rope_fused"] is True and report["ve_rope_fused"] is True
            assert report["flow_cache_hook"] is True and report["decode_graph"] is True

            for name, ref, kw in (("text", ref_text, {}),
                                  ("image", ref_img, dict(pixel_values=px, image_grid_thw=grid))):
                seq, scores = generate(vlm, text_ids if name == "text" else img_ids, **kw)
                print(f"generate {name}: graphs {len(vlm.forward._umic_runner.graphs)} "
                      f"calls {dict(log)}", flush=True)
                assert torch.equal(seq, ref[0]), (name, seq, ref[0])
                err = (scores - ref[1]).abs().max() / ref[1].abs().max()
                assert err <= TOL, (name, float(err))
            vit = visual(px, grid_thw=grid)
            torch.cuda.synchronize()
            for a, b in ((vit.pooler_output, ref_vit.pooler_output),
                         (vit.deepstack_features[0], ref_vit.deepstack_features[0])):
                assert max_rel_err(a, b) <= TOL, max_rel_err(a, b)
            out_exp = expert_steps(expert, prefix, acts)
            for i, (a, b) in enumerate(zip(out_exp, ref_exp)):
                assert torch.equal(a, b), (i, max_rel_err(a, b))
        finally:
            integrate.unfuse_rope()
    print("calls", dict(log), flush=True)
    assert vlm.forward._umic_runner.replays > 0
    for name in ("umic_rmsnorm_bf16", "umic_add_rmsnorm_bf16", "umic_qk_rmsnorm_rope_bf16",
                 "umic_qk_rmsnorm_rope_kv_append_bf16", "umic_linear_multi_bf16",
                 "umic_linear_add_bf16", "umic_gate_silu_mul_bf16", "umic_layernorm_bf16",
                 "umic_add_layernorm_bf16", "umic_rope_qk_bf16"):
        assert log[name] > 0, name
    # the tiled linears at prefill and the ViT's fc1 + GELU, the GEMVs at decode
    assert log["umic_linear_ws_bf16"] + log["umic_linear_bf16"] > 0
