"""CPU: the in-place KV cache (umic.cache) against transformers' DynamicCache.

The in-place cache must be observably the same cache as the concatenating
DynamicCache the reference replaces (src/umic/cache.py): the same keys and
values after every append and crop, the same model outputs when a text model
runs on it, an overflow error instead of a silent grow, and the replay-time
write at a device-held cursor.  Its storage is one arena per layer geometry.  On the CPU the fused-attention patch
(``fuse_kv_rope``) takes its eager branch, so these tests also pin that branch
(RoPE through transformers, then ``update``) against the unpatched model.
"""

from __future__ import annotations

import pytest
import torch
from transformers.cache_utils import DynamicCache, DynamicLayer

from umic import integrate
from umic.cache import InplaceKVCache, InplaceLayer, KVArena

pytestmark = pytest.mark.filterwarnings("ignore::FutureWarning")
BF = torch.bfloat16


def kv(B, H, S, D, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, H, S, D, generator=g).to(BF),
            torch.randn(B, H, S, D, generator=g).to(BF))


def text_model(layers=2):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    cfg = Qwen3VLTextConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                            num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                            vocab_size=64, rope_parameters={"rope_type": "default",
                                                            "rope_theta": 1e6},
                            attn_implementation="sdpa")
    torch.manual_seed(0)
    return Qwen3VLTextModel(cfg).to(BF).eval()


def test_inplace_layer_tracks_dynamic_layer_through_appends_and_crops():
    B, H, D, cap = 2, 3, 16, 40
    ref = DynamicLayer()
    k0, v0 = kv(B, H, 6, D, 0)
    ref.update(k0, v0)
    arena = KVArena(1, B, H, cap, D, BF, "cpu")
    lyr = InplaceLayer(arena, 0)
    lyr.update(k0, v0)
    kb = arena.k(0)
    steps = [("add", 5), ("add", 1), ("crop", 8), ("add", 3), ("crop", -2), ("add", 1),
             ("add", 7), ("crop", 0), ("add", 2)]
    for i, (op, n) in enumerate(steps):
        if op == "add":
            k, v = kv(B, H, n, D, 10 + i)
            rk, rv = ref.update(k, v)
            ik, iv = lyr.update(k, v)
            assert torch.equal(ik, rk) and torch.equal(iv, rv)
            # single-token steps return contiguous copies, longer ones views
            if n == 1:
                assert ik.is_contiguous() and ik.data_ptr() != kb.data_ptr()
            else:
                assert ik.data_ptr() == kb.data_ptr()
        else:
            # crop(n): keep n tokens (n >= 0) or drop -n; DynamicLayer.crop
            # takes the number to drop
            keep = n if n >= 0 else ref.get_seq_length() + n
            if keep < ref.get_seq_length():
                ref.crop(keep - ref.get_seq_length())
            lyr.crop(n)
        assert lyr.get_seq_length() == ref.get_seq_length()
        assert torch.equal(lyr.keys, ref.keys) and torch.equal(lyr.values, ref.values)
    assert lyr.get_max_length() == cap and kb.data_ptr() == arena.storage.data_ptr()


def test_overflow_raises_and_keeps_the_cache():
    arena = KVArena(1, 1, 2, 8, 4, BF, "cpu")
    arena.storage.zero_()
    lyr = InplaceLayer(arena, 0)
    lyr.update(*kv(1, 2, 6, 4, 0))
    k, v = kv(1, 2, 3, 4, 1)
    with pytest.raises(RuntimeError, match="overflow"):
        lyr.update(k, v)
    assert lyr.get_seq_length() == 6 and not arena.k(0)[:, :, 6:].any()
    with pytest.raises(ValueError):
        KVArena(1, 1, 0, 8, 4, BF, "cpu")


def test_arena_layout_one_allocation():
    """Every layer of one geometry lives in one allocation: k and v of a layer
    are adjacent views with equal strides (what the fused append writes)."""
    dyn = DynamicCache()
    for i in range(4):
        dyn.update(*kv(1, 2, 5, 8, i), layer_idx=i)
    conv = InplaceKVCache.from_dynamic(dyn, extra_tokens=3, margin=0)
    assert len(conv.arenas) == 1
    ar = conv.arenas[0]
    assert tuple(ar.storage.shape) == (4, 2, 1, 2, 8, 8)
    for i, lyr in enumerate(conv.layers):
        assert lyr.arena is ar and lyr.index == i
        assert ar.k(i).stride() == ar.v(i).stride()
        assert ar.v(i).data_ptr() - ar.k(i).data_ptr() == ar.k(i).numel() * 2


def test_from_dynamic_copies_the_prefix_once():
    B, H, S, D = 1, 2, 5, 8
    dyn = DynamicCache()
    for i in range(3):
        dyn.update(*kv(B, H, S, D, i), layer_idx=i)
    conv = InplaceKVCache.from_dynamic(dyn, extra_tokens=10, margin=4)
    assert len(conv.layers) == 3 and conv.get_seq_length() == S
    for i, lyr in enumerate(conv.layers):
        assert lyr.capacity == S + 10 + 4
        assert torch.equal(lyr.keys, dyn.layers[i].keys)
        assert torch.equal(lyr.values, dyn.layers[i].values)
        assert lyr.arena.k(lyr.index).data_ptr() != dyn.layers[i].keys.data_ptr()
    conv.update(*kv(B, H, 3, D, 9), layer_idx=1)
    assert conv.get_seq_length(1) == S + 3 and conv.get_seq_length(0) == S
    conv.crop(S)
    assert all(lyr.get_seq_length() == S for lyr in conv.layers)
    assert conv.get_seq_length(7) == 0


def test_replay_writes_at_the_device_cursor():
    B, H, D = 1, 2, 8
    dyn = DynamicCache()
    dyn.update(*kv(B, H, 4, D, 0), layer_idx=0)
    conv = InplaceKVCache.from_dynamic(dyn, extra_tokens=4, margin=0)
    assert conv.layers[0].capacity == 8
    cursor = torch.tensor([6])
    conv.replay_at(cursor, 7)
    k, v = kv(B, H, 1, D, 3)
    rk, rv = conv.update(k, v, 0)
    assert rk.shape[2] == 7 and rk.is_contiguous()
    assert torch.equal(rk[:, :, 6:7], k) and torch.equal(rv[:, :, 6:7], v)
    assert conv.get_seq_length() == 4          # the host fill is set separately
    conv.set_length(7)
    conv.end_replay()
    assert conv.layers[0].keys.shape[2] == 7
    assert torch.equal(conv.layers[0].keys[:, :, 6:7], k)
    # a multi-token write during replay goes to the host fill, as eagerly
    conv.replay_at(cursor, 7)
    conv.update(*kv(B, H, 1, D, 4), 0)
    conv.end_replay()
    conv.update(*kv(B, H, 1, D, 5), 0)
    assert conv.get_seq_length() == 8


def test_reseed_keeps_the_buffers():
    """A new inference with the same prompt length is copied into the same
    arena, so addresses baked into captured graphs stay valid."""
    d1, d2 = DynamicCache(), DynamicCache()
    for i in range(2):
        d1.update(*kv(1, 2, 5, 8, i), layer_idx=i)
        d2.update(*kv(1, 2, 5, 8, 10 + i), layer_idx=i)
    conv = InplaceKVCache.from_dynamic(d1, extra_tokens=4)
    ptr = conv.arenas[0].storage.data_ptr()
    conv.update(*kv(1, 2, 2, 8, 7), layer_idx=0)
    conv.reseed(d2)
    assert conv.arenas[0].storage.data_ptr() == ptr and conv.get_seq_length() == 5
    for a, b in zip(conv.layers, d2.layers):
        assert torch.equal(a.keys, b.keys) and torch.equal(a.values, b.values)


def test_text_model_on_the_inplace_cache_matches_dynamic_cache():
    """Prefill, then an append-then-crop loop (the flow expert's pattern) on
    both caches: hidden states and cache contents agree exactly, with the
    fused-attention patch installed (eager branch on the CPU)."""
    model = text_model()
    torch.manual_seed(1)
    pre = torch.randn(1, 20, 128).to(BF)
    with torch.no_grad():
        dyn = DynamicCache()
        model(inputs_embeds=pre, past_key_values=dyn, use_cache=True)
        conv = InplaceKVCache.from_dynamic(dyn, extra_tokens=8)
        ref_model = text_model()
        assert integrate.fuse_kv_rope(model) == 2
        for step in range(3):
            x = torch.randn(1, 8, 128).to(BF)
            ref = ref_model(inputs_embeds=x, past_key_values=dyn, use_cache=True)
            out = model(inputs_embeds=x, past_key_values=conv, use_cache=True)
            assert torch.equal(out.last_hidden_state, ref.last_hidden_state), step
            for a, b in zip(conv.layers, dyn.layers):
                assert torch.equal(a.keys, b.keys) and torch.equal(a.values, b.values)
            dyn.crop(-8)
            conv.crop(20)
    assert integrate.unfuse_mlps(model) == 2


def test_fuse_repeat_cache_substitutes_once_and_resyncs():
    model = text_model(layers=1)
    seen = []

    class Expert(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.lm = model

        def forward(self, inputs_embeds=None, past_key_values=None):
            seen.append(past_key_values)
            return self.lm(inputs_embeds=inputs_embeds, past_key_values=past_key_values,
                           use_cache=True)

    expert = Expert()
    integrate.fuse_repeat_cache(expert, extra_tokens_hint=4)
    torch.manual_seed(2)
    with torch.no_grad():
        dyn = DynamicCache()
        model(inputs_embeds=torch.randn(1, 10, 128).to(BF), past_key_values=dyn, use_cache=True)
        for _ in range(2):
            expert(inputs_embeds=torch.randn(1, 6, 128).to(BF), past_key_values=dyn)
    assert isinstance(seen[0], InplaceKVCache) and seen[1] is seen[0]
    # the caller's cache is untouched; the substitute was cropped back to it
    assert dyn.get_seq_length() == 10 and seen[0].get_seq_length() == 16
    assert seen[0].layers[0].capacity == 10 + 6 + 8


def test_decode_graph_runner_passes_cpu_calls_through():
    """On CPU tensors the runner is a pass-through: generate() is unchanged
    and nothing is captured."""
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLForConditionalGeneration

    from umic.graph import DecodeGraphRunner

    cfg = Qwen3VLConfig(
        text_config=dict(hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                         vocab_size=256, rope_parameters={"rope_type": "default",
                                                          "rope_theta": 1e6,
                                                          "mrope_section": [8, 4, 4],
                                                          "mrope_interleaved": True}),
        vision_config=dict(depth=1, hidden_size=64, num_heads=4, intermediate_size=128,
                           out_hidden_size=128, patch_size=4, temporal_patch_size=2,
                           spatial_merge_size=2, num_position_embeddings=64,
                           deepstack_visual_indexes=[]))
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    m = Qwen3VLForConditionalGeneration(cfg).to(BF).eval()
    ids = torch.randint(0, 256, (1, 12), generator=torch.Generator().manual_seed(3))
    kw = dict(input_ids=ids, attention_mask=torch.ones_like(ids), max_new_tokens=4,
              do_sample=False)
    with torch.no_grad():
        ref = m.generate(**kw)
        runner = DecodeGraphRunner(m, max_new_tokens=8)
        out = m.generate(**kw)
    assert torch.equal(out, ref)
    assert runner.replays == 0 and not len(runner.graphs) and runner.cache is None


def test_flow_step_graph_falls_back_to_eager_on_cpu():
    """FlowStepGraph on CPU tensors: capture is unavailable, so after the
    warm-up steps it falls back to eager for good, with the same results;
    fuse_flow_graph wraps the step closures handed to diffusion.sample."""
    from umic.graph import FlowStepGraph, fuse_flow_graph

    calls = []

    def step_fn(x, t):
        calls.append(1)
        return x * 2 + t

    fsg = FlowStepGraph(step_fn, warmup=2)
    xs = [torch.randn(1, 4, 8) for _ in range(5)]
    for i, x in enumerate(xs):
        t = torch.full((1,), float(i))
        assert torch.equal(fsg(x, t), x * 2 + t)
    assert fsg.disabled and not fsg.captured and len(calls) == 5

    class Diffusion:
        def sample(self, noise, step_fn=None, unguided_step_fn=None):
            self.seen = (step_fn, unguided_step_fn)
            return step_fn(x=noise, t=torch.zeros(1))

    model = torch.nn.Module()
    model.diffusion = Diffusion()
    fuse_flow_graph(model)
    x = torch.randn(2, 3)
    assert torch.equal(model.diffusion.sample(x, step_fn=step_fn), x * 2)
    assert isinstance(model.diffusion.seen[0], FlowStepGraph) and model.diffusion.seen[1] is None


def test_repeat_cache_rebinds_to_a_new_cache_object():
    """A second inference's cache -- freed and rebuilt, same length, possibly
    at the freed cache's address -- gets a fresh stand-in: the expert sees the
    new prefix, never the previous inference's KV."""
    import gc

    from umic.cache import CacheStandIn

    model = text_model(layers=1)
    seen = []

    class Expert(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.lm = model

        def forward(self, inputs_embeds=None, past_key_values=None):
            seen.append(past_key_values)
            return self.lm(inputs_embeds=inputs_embeds, past_key_values=past_key_values,
                           use_cache=True)

    expert = Expert()
    integrate.fuse_repeat_cache(expert, extra_tokens_hint=4)
    integrate.fuse_repeat_cache(expert, extra_tokens_hint=4)   # idempotent
    assert len(expert._forward_pre_hooks) == 1
    stand_in = expert._umic_cache_stand_in
    assert isinstance(stand_in, CacheStandIn)

    def prefix(seed):
        torch.manual_seed(seed)
        dyn = DynamicCache()
        with torch.no_grad():
            model(inputs_embeds=torch.randn(1, 10, 128).to(BF), past_key_values=dyn,
                  use_cache=True)
        return dyn

    step = torch.randn(1, 6, 128).to(BF)
    dyn = prefix(3)
    with torch.no_grad():
        expert(inputs_embeds=step, past_key_values=dyn)
    first = seen[-1]
    del dyn
    gc.collect()
    dyn2 = prefix(4)
    want = [lyr.keys.clone() for lyr in dyn2.layers]
    with torch.no_grad():
        expert(inputs_embeds=step, past_key_values=dyn2)
    second = seen[-1]
    assert second is not first and stand_in.bound_to(dyn2)
    for lyr, k in zip(second.layers, want):
        assert torch.equal(lyr.keys[:, :, :10], k)
    # the same object again: the stand-in is reused and cut back to 10 tokens
    with torch.no_grad():
        expert(inputs_embeds=step, past_key_values=dyn2)
    assert seen[-1] is second and second.get_seq_length() == 16
    # nothing to stand in for: no cache, a stand-in already, empty layers
    assert stand_in.resolve(None) is None and stand_in.resolve(second) is None
    assert stand_in.resolve(DynamicCache()) is None
