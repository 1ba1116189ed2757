"""GPU: decode-step and flow-step HIP graphs (umic.graph).

DecodeGraphRunner, on a small random-weight Qwen3-VL, text-only prompts,
greedy generate():

The same prompts are decoded eagerly by the unpatched model first; then the
LM gets the fused kernels (RMSNorm, add+RMSNorm, text RoPE, RoPE + in-place
KV append, the q/k/v projections as one GEMV launch, q/o GEMVs, the P5 MLP
GEMV with the residual add in down_proj's epilogue) and the runner, and every
generation must produce the eager tokens, with per-step scores equal within
bf16 noise.  Four inferences: the
first warms up for two steps and captures one graph per remaining KV length,
the second (same prompt length, new prompt, on the persistent buffers)
captures the two warm-up lengths, the third is pure replay, the fourth (new
prompt length) warms up and recaptures.  Replays run with generate()'s own eager work (sampling)
and synchronisations between them.  Attention is held to the flash /
memory-efficient SDPA kernels (q and kv head counts equal, so no
grouped-query support is needed): an unsupported case raises rather than
running the bf16 math path.
"""

from __future__ import annotations

import collections

import pytest
import torch

from umic import _lib, integrate
from umic.graph import DecodeGraphRunner

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::FutureWarning"),
              pytest.mark.filterwarnings("ignore::UserWarning")]
DEV = "cuda"
NEW = 10


def small_vlm():
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLForConditionalGeneration

    cfg = Qwen3VLConfig(
        text_config=dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=4, head_dim=128,
                         vocab_size=512, rope_parameters={"rope_type": "default",
                                                          "rope_theta": 1e6,
                                                          "mrope_section": [24, 20, 20],
                                                          "mrope_interleaved": True}),
        vision_config=dict(depth=1, hidden_size=64, num_heads=4, intermediate_size=128,
                           out_hidden_size=256, patch_size=4, temporal_patch_size=2,
                           spatial_merge_size=2, num_position_embeddings=64,
                           deepstack_visual_indexes=[]))
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    m = Qwen3VLForConditionalGeneration(cfg)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.copy_(1 + 0.1 * torch.randn_like(p))
    return m.to(torch.bfloat16).to(DEV).eval()


def generate(m, ids):
    out = m.generate(input_ids=ids, attention_mask=torch.ones_like(ids), max_new_tokens=NEW,
                     do_sample=False, output_scores=True, return_dict_in_generate=True)
    torch.cuda.synchronize()
    return out.sequences.cpu(), torch.stack(out.scores).float().cpu()


def test_decode_graph_runner_matches_eager(monkeypatch):
    from torch.nn.attention import SDPBackend, sdpa_kernel

    m = small_vlm()
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, 512, (1, n), generator=g).to(DEV) for n in (24, 24, 24, 17)]
    with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION,
                                       SDPBackend.EFFICIENT_ATTENTION]):
        ref = [generate(m, p) for p in prompts]
        lm = m.model.language_model
        assert integrate.fuse_rmsnorms(lm) > 0 and integrate.fuse_add_rmsnorm(lm) == 2
        assert integrate.fuse_text_rope() and integrate.fuse_kv_rope(lm) == 2
        assert integrate.fuse_mlps(lm) == 2 and integrate.fuse_linears(lm) == 4
        runner = DecodeGraphRunner(m, max_new_tokens=NEW)
        log = collections.Counter()
        real = _lib.call

        def spy(name, *args):
            log[name] += 1
            return real(name, *args)

        monkeypatch.setattr(_lib, "call", spy)
        try:
            captured = []
            for i, p in enumerate(prompts):
                seq, scores = generate(m, p)
                captured.append(len(runner.graphs))
                print(f"inference {i}: prompt {p.shape[1]} graphs {len(runner.graphs)} "
                      f"replays {runner.replays} calls {dict(log)}", flush=True)
                assert torch.equal(seq, ref[i][0]), (i, seq, ref[i][0])
                err = (scores - ref[i][1]).abs().max() / ref[i][1].abs().max()
                assert err <= 2e-2, (i, float(err))
        finally:
            integrate.unfuse_rope()
            integrate.unfuse_mlps(lm)
    # NEW - 1 decode steps per inference (the first token comes from prefill);
    # with no graphs yet, the first two steps are eager warm-up
    assert captured == [NEW - 3, NEW - 1, NEW - 1, NEW - 3]
    assert runner.replays == (NEW - 3) + (NEW - 1) + (NEW - 1) + (NEW - 3)
    # q/k norms, RoPE and the append ran fused in the graphs, norms and RoPE
    # fused at prefill
    assert log["umic_qk_rmsnorm_rope_kv_append_bf16"] > 0
    assert log["umic_qk_rmsnorm_rope_bf16"] > 0
    # the decode GEMVs: q/k/v in one launch, the P5 MLP, down_proj + residual
    for name in ("umic_linear_multi_bf16", "umic_gate_silu_mul_bf16", "umic_linear_add_bf16"):
        assert log[name] > 0, name


def test_flow_step_graph_replays_match_eager():
    """FlowStepGraph over a flow-expert-like step: 32 action tokens through a
    config-5 decoder layer that appends to an in-place KV cache (q/k norms,
    RoPE and the append fused) and attends to the whole prefix, then crops back.  Ten
    steps with new x and t: each replay equals the eager step bit for bit,
    and the cache prefix is untouched."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from transformers.cache_utils import DynamicCache

    from helpers import qwen3_decoder_layer
    from umic.cache import InplaceKVCache
    from umic.graph import FlowStepGraph

    layer, rot = qwen3_decoder_layer(DEV)
    P, N = 1024, 32
    torch.manual_seed(11)
    h0 = torch.randn(1, P, 4096).to(torch.bfloat16).to(DEV)
    with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION,
                                       SDPBackend.EFFICIENT_ATTENTION]):
        dyn = DynamicCache()
        layer(h0, position_embeddings=rot(h0, torch.arange(P, device=DEV)[None]),
              past_key_values=dyn)
        cache = InplaceKVCache.from_dynamic(dyn, extra_tokens=N)
        prefix_k = cache.layers[0].keys.clone()
        assert integrate.fuse_kv_rope(layer) == 1
        cs = rot(h0[:, :N], torch.arange(P, P + N, device=DEV)[None])

        def step_fn(x, t):
            out = layer(x + t, position_embeddings=cs, past_key_values=cache, is_causal=False)
            cache.crop(P)
            return out

        fsg = FlowStepGraph(step_fn, warmup=2)
        g = torch.Generator().manual_seed(12)
        for i in range(10):
            x = torch.randn(1, N, 4096, generator=g).to(torch.bfloat16).to(DEV)
            t = torch.full((1, 1, 1), 0.1 * i).to(torch.bfloat16).to(DEV)
            ref = step_fn(x=x, t=t)
            out = fsg(x, t)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), i
        assert fsg.captured and not fsg.disabled
        assert torch.equal(cache.arenas[0].k(0)[:, :, :P], prefix_k)
    integrate.unfuse_mlps(layer)
