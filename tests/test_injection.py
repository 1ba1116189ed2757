"""Injection semantics on real transformers module trees, on the CPU.

Mirrors the reference's structural contract (src/umic/integrate.py,
src/umic/optimize.py): duck-typed matching with dry-run counts, forward
swap by instance attribute, weights shared (no copy), non-matching models
untouched, FUSE_MIN_ROWS regime dispatch for the GEMM sites, idempotent
RoPE swaps, and the original eager math for every input the fused kernels
do not take (here: CPU tensors) -- bit-identical to the unpatched model.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from umic import integrate, optimize
from umic.kernels import fused_ffn, linear

pytestmark = pytest.mark.filterwarnings("ignore::FutureWarning")

BF = torch.bfloat16


def tiny_text_model(layers=2, dtype=BF):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    cfg = Qwen3VLTextConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                            num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                            vocab_size=64, rope_parameters={"rope_type": "default",
                                                            "rope_theta": 1e6},
                            attn_implementation="sdpa")
    torch.manual_seed(0)
    return Qwen3VLTextModel(cfg).to(dtype).eval()


def tiny_vision_model(dtype=BF):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLVisionConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLVisionModel

    cfg = Qwen3VLVisionConfig(depth=4, hidden_size=64, num_heads=4, intermediate_size=128,
                              patch_size=4, temporal_patch_size=2, in_channels=3,
                              spatial_merge_size=2, out_hidden_size=96,
                              num_position_embeddings=64, deepstack_visual_indexes=[1],
                              attn_implementation="sdpa")
    torch.manual_seed(0)
    m = Qwen3VLVisionModel(cfg).to(dtype).eval()
    with torch.no_grad():  # non-trivial LayerNorm affine params
        for mod in m.modules():
            if isinstance(mod, nn.LayerNorm):
                mod.weight.add_(0.1 * torch.randn_like(mod.weight))
                mod.bias.add_(0.1 * torch.randn_like(mod.bias))
    return m


def text_inputs(model, S=80, dtype=BF):
    torch.manual_seed(1)
    h = torch.randn(1, S, model.config.hidden_size).to(dtype)
    pos = torch.arange(S)[None]
    return dict(inputs_embeds=h, position_ids=pos)


@pytest.fixture(autouse=True)
def _restore_rope():
    yield
    integrate.unfuse_rope()


# ---- matching and counts ---------------------------------------------------

def test_dry_run_counts_and_no_patch():
    m = tiny_text_model()
    assert integrate.fuse_mlps(m, dry_run=True) == 2
    assert integrate.fuse_linears(m, dry_run=True) == 4       # q_proj, o_proj x 2
    assert integrate.fuse_rmsnorms(m, dry_run=True) == 9      # 4 per layer + final
    assert integrate.fuse_add_rmsnorm(m, dry_run=True) == 2
    assert not any("forward" in mod.__dict__ for mod in m.modules())


def test_patch_binds_instance_forward_and_unfuse_restores():
    m = tiny_text_model()
    n = (integrate.fuse_mlps(m) + integrate.fuse_linears(m) + integrate.fuse_rmsnorms(m)
         + integrate.fuse_add_rmsnorm(m))
    patched = [mod for mod in m.modules() if "forward" in mod.__dict__]
    assert len(patched) == n == 17
    assert m.layers[0].mlp.forward.__func__ is integrate._fused_mlp_forward
    assert integrate.unfuse_mlps(m) == 17
    assert not any("forward" in mod.__dict__ for mod in m.modules())


def test_weights_shared_not_copied():
    m = tiny_text_model()
    before = {k: (v.data_ptr(), v.clone()) for k, v in m.state_dict().items()}
    optimize.apply(_wrap(lm=m))
    for k, v in m.state_dict().items():
        assert v.data_ptr() == before[k][0], k
        assert torch.equal(v, before[k][1]), k


def test_non_matching_model_is_noop():
    m = nn.Sequential(nn.Linear(8, 8), nn.ReLU(), nn.LayerNorm(8, elementwise_affine=False))
    assert integrate.fuse_mlps(m) == 0
    assert integrate.fuse_linears(m) == 0
    assert integrate.fuse_rmsnorms(m) == 0
    assert integrate.fuse_add_rmsnorm(m) == 0
    assert integrate.fuse_layernorms(m) == 0
    assert integrate.fuse_vision_encoder_pipeline(m) == 0
    assert not any("forward" in mod.__dict__ for mod in m.modules())
    report = optimize.apply(m)  # no .vlm: LM fusions skipped, nothing patched
    assert all(v in (False, True) for v in report.values())
    assert not any("forward" in mod.__dict__ for mod in m.modules())


def test_p5_matcher_rules():
    class MLP(nn.Module):
        def __init__(self, act, bias=False):
            super().__init__()
            self.gate_proj = nn.Linear(8, 16, bias=bias)
            self.up_proj = nn.Linear(8, 16, bias=False)
            self.down_proj = nn.Linear(16, 8, bias=False)
            self.act_fn = act

    assert integrate._is_p5_mlp(MLP(nn.SiLU()))
    assert not integrate._is_p5_mlp(MLP(nn.GELU()))
    assert not integrate._is_p5_mlp(MLP(nn.SiLU(), bias=True))


# ---- eager fallback is the original math, bit for bit ----------------------

def test_cpu_patched_text_model_is_bit_identical():
    m = tiny_text_model()
    inp = text_inputs(m)
    with torch.no_grad():
        ref = m(**inp).last_hidden_state
        integrate.fuse_mlps(m)
        integrate.fuse_linears(m)
        integrate.fuse_rmsnorms(m)
        integrate.fuse_add_rmsnorm(m)
        assert integrate.fuse_text_rope()
        out = m(**inp).last_hidden_state
    assert torch.equal(out, ref)


def test_cpu_patched_vision_model_is_bit_identical():
    m = tiny_vision_model()
    cfg = m.config
    grid = torch.tensor([[1, 4, 6], [1, 2, 2]])
    n_patch = int((grid[:, 0] * grid[:, 1] * grid[:, 2]).sum())
    torch.manual_seed(2)
    px = torch.randn(n_patch, cfg.in_channels * cfg.temporal_patch_size * cfg.patch_size**2)
    with torch.no_grad():
        ref = m(px.to(BF), grid_thw=grid)
        assert integrate.fuse_layernorms(m) == 4 * 2 + 1 + 1   # blocks, merger, deepstack merger
        assert integrate.fuse_vision_rope()
        assert integrate.fuse_vision_encoder_pipeline(m) == 1
        assert integrate.fuse_gelu_mlps(m) == 4      # blocks; not the mergers
        out = m(px.to(BF), grid_thw=grid)
        out2 = m(px.to(BF), grid_thw=grid)  # cached constants path
    for o in (out, out2):
        assert torch.equal(o.last_hidden_state, ref.last_hidden_state)
        assert torch.equal(o.pooler_output, ref.pooler_output)
        assert len(o.deepstack_features) == len(ref.deepstack_features) == 1
        assert torch.equal(o.deepstack_features[0], ref.deepstack_features[0])
    assert len(m._umic_ve_cache) == 2


# ---- FUSE_MIN_ROWS regime dispatch ----------------------------------------

def test_fuse_min_rows_boundary(monkeypatch):
    """Decode-sized calls take the library's GEMV up to each site's measured
    limit (P5 and q/o_proj 4 rows, the MLP's down projection 2); from there
    the vendor path, until a site's tiled kernel wins: P5 from 256 rows, the
    plain q/o linear never."""
    calls = []

    def fake_p5(x, wg_kn, wu_kn):
        calls.append(("p5", x.reshape(-1, x.shape[-1]).shape[0]))
        return fused_ffn.gate_silu_mul_eager(x, wg_kn, wu_kn)

    def fake_lin(x, w, b=None, act=None):
        calls.append(("lin", x.reshape(-1, x.shape[-1]).shape[0]))
        return nn.functional.linear(x, w, b)

    monkeypatch.setattr(fused_ffn, "p5_eligible", lambda *a: True)
    monkeypatch.setattr(fused_ffn, "gate_silu_mul_hip", fake_p5)
    monkeypatch.setattr(linear, "linear_eligible", lambda *a: True)
    monkeypatch.setattr(linear, "linear_hip", fake_lin)
    m = tiny_text_model(layers=1)
    integrate.fuse_mlps(m)
    integrate.fuse_linears(m)
    mlp, q = m.layers[0].mlp, m.layers[0].self_attn.q_proj
    for rows in (2, 3, 4, 5, 8, 63, 64, 255, 256):
        x = torch.randn(1, rows, 128).to(BF)
        with torch.no_grad():
            mlp(x)
            q(x)
    assert calls == [("p5", 2), ("lin", 2), ("lin", 2), ("p5", 3), ("lin", 3), ("p5", 4),
                     ("lin", 4), ("p5", 256)]
    assert integrate.FUSE_MIN_ROWS == 64 and integrate.GEMV_MAX_ROWS == 8
    assert (integrate.GEMV_ROWS_MLP, integrate.GEMV_ROWS_LINEAR,
            integrate.GEMV_ROWS_DOWN) == (4, 4, 2)
    assert (integrate.TILED_MIN_ROWS_MLP, integrate.TILED_MIN_ROWS_LINEAR) == (256, None)
    # a site's tiled kernel can be re-enabled from a chosen row count
    monkeypatch.setattr(integrate, "TILED_MIN_ROWS_LINEAR", 64)
    calls.clear()
    with torch.no_grad():
        q(torch.randn(1, 64, 128).to(BF))
        q(torch.randn(1, 63, 128).to(BF))
    assert calls == [("lin", 64)]


def test_gelu_mlp_min_rows_and_activation_kind(monkeypatch):
    """The ViT MLP's fc1 takes the fused linear from TILED_MIN_ROWS_GELU_MLP
    (2048) rows, where it stops losing to the vendor path, with the GELU form
    the module computes (Qwen3-VL's ViT: gelu_pytorch_tanh)."""
    calls = []

    def fake_lin(x, w, b=None, act=None):
        calls.append((x.reshape(-1, x.shape[-1]).shape[0], act))
        h = nn.functional.linear(x, w, b)
        return nn.functional.gelu(h, approximate="tanh" if act == "gelu_tanh" else "none")

    monkeypatch.setattr(linear, "linear_eligible", lambda *a: True)
    monkeypatch.setattr(linear, "linear_hip", fake_lin)
    m = tiny_vision_model()
    integrate.fuse_gelu_mlps(m)
    mlp = m.blocks[0].mlp
    for rows in (64, 2047, 2048):
        with torch.no_grad():
            mlp(torch.randn(rows, 64).to(BF))
    assert calls == [(2048, "gelu_tanh")]


def test_autograd_keeps_the_eager_path(monkeypatch):
    """The kernels have no backward: with grad mode on and weights that
    require grad, every GEMM and norm site runs the class forward (autograd
    records eager's graph); under no_grad the same calls take the kernels."""
    from umic.kernels import rmsnorm

    calls = []

    def fake_p5(x, wg_kn, wu_kn):
        calls.append("p5")
        return fused_ffn.gate_silu_mul_eager(x, wg_kn, wu_kn)

    def fake_lin(x, w, b=None, act=None):
        calls.append("lin")
        return nn.functional.linear(x, w, b)

    def fake_rms(x, w, eps):
        calls.append("rms")
        return x

    monkeypatch.setattr(fused_ffn, "p5_eligible", lambda *a: True)
    monkeypatch.setattr(fused_ffn, "gate_silu_mul_hip", fake_p5)
    monkeypatch.setattr(linear, "linear_eligible", lambda *a: True)
    monkeypatch.setattr(linear, "linear_hip", fake_lin)
    monkeypatch.setattr(rmsnorm, "rmsnorm_eligible", lambda *a: True)
    monkeypatch.setattr(rmsnorm, "rmsnorm_hip", fake_rms)
    m = tiny_text_model(layers=1)
    integrate.fuse_mlps(m)
    integrate.fuse_linears(m)
    integrate.fuse_rmsnorms(m)
    mlp, q, norm = m.layers[0].mlp, m.layers[0].self_attn.q_proj, m.norm
    x = torch.randn(1, 4, 128).to(BF)  # the GEMV regime of P5 and q_proj
    assert mlp.gate_proj.weight.requires_grad
    out = mlp(x)
    q(x)
    norm(x)
    assert calls == [] and out.requires_grad
    out.float().sum().backward()
    assert mlp.gate_proj.weight.grad is not None
    with torch.no_grad():
        mlp(x)
        q(x)
        norm(x)
    assert calls == ["p5", "lin", "rms"]
    with torch.inference_mode():
        norm(x)
    assert calls[-1] == "rms" and len(calls) == 4


def test_gelu_kind_by_values():
    from transformers import activations as hf

    assert integrate._gelu_kind(nn.GELU()) == "gelu"
    assert integrate._gelu_kind(nn.GELU(approximate="tanh")) == "gelu_tanh"
    assert integrate._gelu_kind(nn.functional.gelu) == "gelu"
    assert integrate._gelu_kind(hf.GELUActivation()) == "gelu"
    assert integrate._gelu_kind(hf.ACT2FN["gelu_pytorch_tanh"]) == "gelu_tanh"
    assert integrate._gelu_kind(hf.NewGELUActivation()) == "gelu_tanh"
    # GELU-named but another function: left to eager
    assert integrate._gelu_kind(hf.QuickGELUActivation()) is None
    assert integrate._gelu_kind(nn.SiLU()) is None
    assert integrate._gelu_kind(None) is None


class _ToyMLP(nn.Module):
    def forward(self, x):
        return self.fc2(self.act_fn(self.fc1(x)))


def test_gelu_mlp_matcher_rules():
    def mlp(d_in=32, d_hid=64, d_out=32, act=None, gate=False, names=("fc1", "fc2")):
        m = _ToyMLP()
        setattr(m, names[0], nn.Linear(d_in, d_hid))
        setattr(m, names[1], nn.Linear(d_hid, d_out))
        m.act_fn = act if act is not None else nn.GELU()
        if gate:
            m.gate_proj = nn.Linear(d_in, d_hid)
        return m

    assert integrate._is_gelu_mlp(mlp())[2] == "gelu"
    assert integrate._is_gelu_mlp(mlp(names=("linear_fc1", "linear_fc2")))[2] == "gelu"
    assert integrate._is_gelu_mlp(mlp(act=nn.GELU(approximate="tanh")))[2] == "gelu_tanh"
    assert integrate._is_gelu_mlp(mlp(d_out=48)) is None          # patch-merger shape
    assert integrate._is_gelu_mlp(mlp(gate=True)) is None         # a gated MLP
    assert integrate._is_gelu_mlp(mlp(act=nn.SiLU())) is None
    assert integrate._is_gelu_mlp(mlp(names=("w1", "w2"))) is None
    m = mlp()
    w = m.fc1.weight
    assert integrate.fuse_gelu_mlps(m, dry_run=True) == 1 and "forward" not in m.__dict__
    assert integrate.fuse_gelu_mlps(m) == 1 and m.fc1.weight is w
    x = torch.randn(4, 32)
    assert torch.equal(m(x), m.fc2(m.act_fn(m.fc1(x))))          # CPU: eager


def test_gate_silu_mul_cpu_is_eager():
    torch.manual_seed(3)
    x = torch.randn(16, 64).to(BF)
    wg, wu = torch.randn(32, 64).to(BF), torch.randn(32, 64).to(BF)
    assert torch.equal(fused_ffn.gate_silu_mul(x, wg.t(), wu.t()),
                       fused_ffn.gate_silu_mul_eager(x, wg.t(), wu.t()))


# ---- RoPE swap --------------------------------------------------------------

def test_text_rope_swap_is_idempotent_and_falls_back():
    from transformers.models.qwen3_vl import modeling_qwen3_vl as hf

    orig = hf.apply_rotary_pos_emb
    assert integrate.fuse_text_rope() and integrate.fuse_text_rope()
    fused = hf.apply_rotary_pos_emb
    assert fused is not orig and fused.__wrapped__ is orig and fused._umic_fused
    torch.manual_seed(4)
    q = torch.randn(2, 3, 5, 16).to(BF)     # B = 2, [B, H, S, D]
    cos, sin = torch.randn(2, 5, 16).to(BF), torch.randn(2, 5, 16).to(BF)
    for kw in ({}, {"unsqueeze_dim": 1}):
        a = fused(q, q, cos, sin, **kw)
        b = orig(q, q, cos, sin, **kw)
        assert all(torch.equal(x, y) for x, y in zip(a, b))
    qs = q.transpose(1, 2)                   # [B, S, H, D] with unsqueeze_dim=2
    a, b = fused(qs, qs, cos, sin, unsqueeze_dim=2), orig(qs, qs, cos, sin, unsqueeze_dim=2)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    assert integrate.unfuse_rope() == 1 and hf.apply_rotary_pos_emb is orig


def test_vision_rope_swap_falls_back_on_cpu():
    from transformers.models.qwen3_vl import modeling_qwen3_vl as hf

    orig = hf.apply_rotary_pos_emb_vision
    assert integrate.fuse_vision_rope()
    torch.manual_seed(5)
    q = torch.randn(10, 2, 20).to(BF)
    cos, sin = torch.randn(10, 20), torch.randn(10, 20)
    a, b = hf.apply_rotary_pos_emb_vision(q, q, cos, sin), orig(q, q, cos, sin)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


# ---- apply() ---------------------------------------------------------------

def _wrap(lm=None, visual=None, expert=None):
    vlm = nn.Module()
    if lm is not None:
        vlm.language_model = lm
    if visual is not None:
        vlm.visual = visual
    root = nn.Module()
    root.vlm = vlm
    if expert is not None:
        root.expert = expert
    return root


def test_apply_report():
    model = _wrap(lm=tiny_text_model(), visual=tiny_vision_model(),
                  expert=tiny_text_model(layers=1))
    report = optimize.apply(model)
    assert report["lm_mlp_fused"] == 2 and report["lm_linear_fused"] == 4
    assert report["lm_rmsnorm_fused"] == 9 and report["lm_add_rmsnorm_fused"] == 2
    assert report["text_rope_fused"] is True
    assert report["ve_layernorm_fused"] == 10 and report["ve_rope_fused"] is True
    assert report["ve_pipeline_fused"] == 1 and report["ve_gelu_mlp_fused"] == 4
    assert report["expert_rmsnorm_fused"] == 5 and report["expert_add_rmsnorm_fused"] == 1
    assert report["lm_kv_rope_fused"] == 2 and report["expert_kv_rope_fused"] == 1
    assert report["flow_cache_hook"] is True and report["decode_graph"] is True
    assert "decode_cache_hook" not in report and "adaptive_flow" not in report
    # application order: the reference's (LM, text RoPE, ViT, expert, VLM), with
    # this runtime's additions next to the fusion each extends
    assert list(report) == [
        "lm_mlp_fused", "lm_linear_fused", "lm_rmsnorm_fused", "lm_add_rmsnorm_fused",
        "text_rope_fused", "lm_kv_rope_fused", "ve_layernorm_fused", "ve_rope_fused",
        "ve_pipeline_fused", "ve_gelu_mlp_fused", "flow_cache_hook", "expert_rmsnorm_fused",
        "expert_add_rmsnorm_fused", "expert_kv_rope_fused", "decode_graph"]
    cfg = optimize.UmicConfig(mlp_fusion=False, vision_fusion=False, decode_graph=False,
                              flow_cache=False, decode_cache=False)
    report2 = optimize.apply(_wrap(lm=tiny_text_model()), cfg)
    assert "lm_mlp_fused" not in report2 and "ve_layernorm_fused" not in report2
    assert "decode_graph" not in report2 and "decode_cache_hook" not in report2
    report3 = optimize.apply(_wrap(lm=tiny_text_model()),
                             optimize.UmicConfig(decode_graph=False, adaptive_flow=True))
    assert report3["decode_cache_hook"] is True and report3["adaptive_flow"] is False
    # the expert's fusions follow flow_cache (the reference nests them under it)
    report4 = optimize.apply(_wrap(lm=tiny_text_model(), expert=tiny_text_model(layers=1)),
                             optimize.UmicConfig(flow_cache=False))
    assert not [k for k in report4 if k.startswith(("expert_", "flow_cache"))]
    assert report4["lm_rmsnorm_fused"] == 9
    integrate.unfuse_rope()


def test_apply_twice_is_idempotent():
    """A second apply() patches nothing new: same report, one cache hook per
    module, one decode-graph runner."""
    model = _wrap(lm=tiny_text_model(), visual=tiny_vision_model(),
                  expert=tiny_text_model(layers=1))
    first = optimize.apply(model)
    runner = model.vlm.forward._umic_runner
    hooks = len(model.expert._forward_pre_hooks)
    second = optimize.apply(model)
    assert second == first
    assert model.vlm.forward._umic_runner is runner
    assert runner.wrapped_forward.__self__ is model.vlm
    assert len(model.expert._forward_pre_hooks) == hooks == 1
    integrate.unfuse_rope()


def test_find_lm_module_variants():
    lm = tiny_text_model(layers=1)
    assert optimize.find_lm_module(_wrap(lm=lm)) is lm
    outer = nn.Module()
    outer.model = lm
    root = nn.Module()
    root.vlm = nn.Module()
    root.vlm.language_model = outer
    assert optimize.find_lm_module(root) is outer
    assert optimize.find_lm_module(nn.Linear(2, 2)) is None
    # transformers >= 5: vlm.model is the VLM trunk holding language_model / visual
    vis = tiny_vision_model()
    trunk = nn.Module()
    trunk.language_model, trunk.visual = lm, vis
    root5 = nn.Module()
    root5.vlm = nn.Module()
    root5.vlm.model = trunk
    assert optimize.find_lm_module(root5) is lm
    assert optimize.find_visual_module(root5) is vis
    assert optimize.find_visual_module(_wrap(visual=vis)) is vis


def test_decode_paths_defer_to_hooked_modules():
    """The decode paths call kernels in place of submodule calls only while
    no forward hook would be skipped: a module hook, a pre-hook or a global
    hook sends them back through the module's own __call__."""
    lm = tiny_text_model()
    attn, mlp = lm.layers[0].self_attn, lm.layers[0].mlp
    assert not integrate._hooked(attn.q_proj, mlp, mlp.down_proj)
    seen = []
    h = attn.k_proj.register_forward_hook(lambda m, a, o: seen.append(m))
    assert integrate._hooked(attn.q_proj, attn.k_proj) and not integrate._hooked(attn.q_proj)
    h.remove()
    h = mlp.register_forward_pre_hook(lambda m, a: None)
    assert integrate._hooked(mlp, mlp.down_proj)
    h.remove()
    g = nn.modules.module.register_module_forward_hook(lambda m, a, o: None)
    try:
        assert integrate._hooked(attn.q_proj)
    finally:
        g.remove()
    assert not integrate._hooked(attn.q_proj, attn.k_proj, mlp, mlp.down_proj)
    # a hooked projection still fires on the fused attention path
    assert integrate.fuse_kv_rope(lm) == 2
    h = attn.k_proj.register_forward_hook(lambda m, a, o: seen.append(m))
    with torch.no_grad():
        lm(input_ids=torch.arange(6)[None])
    h.remove()
    integrate.unfuse_mlps(lm)
    assert seen == [attn.k_proj]


def test_kernel_registry():
    """The reference's registry surface (src/umic/kernels/__init__.py:14-23),
    pre-populated with the HIP wrappers; a registration replaces an entry."""
    from umic import kernels
    from umic.kernels import layernorm, rmsnorm, rope

    assert kernels.get_kernel("rmsnorm") is rmsnorm.rmsnorm_hip
    assert kernels.get_kernel("add_layernorm") is layernorm.add_layernorm_hip
    assert kernels.get_kernel("rope_vision") is rope.apply_rotary_vision_hip
    assert kernels.get_kernel("gate_silu_mul") is fused_ffn.gate_silu_mul_hip
    assert kernels.get_kernel("linear") is linear.linear_hip
    assert kernels.get_kernel("no_such_pattern") is None
    mine = lambda *a: None  # noqa: E731
    kernels.register_kernel("rmsnorm", mine)
    try:
        assert kernels.get_kernel("rmsnorm") is mine
    finally:
        kernels.register_kernel("rmsnorm", rmsnorm.rmsnorm_hip)


def test_gemv_norm_plan_matches_torch_reduce_config():
    """The folded-norm plan restates Reduce.cuh's setReduceConfig: at one row
    and n = 4096, 512 threads with two 4-vectors each; two rows split the
    block, 256 threads with four; short rows (< 128 threads) and long rows
    (16+ values per thread: the row would be split over the block) are not
    the wide plan."""
    from umic.kernels import rmsnorm

    assert rmsnorm.wide_plan(1, 4096) == (512, 2)
    assert rmsnorm.wide_plan(2, 4096) == (256, 4)
    assert rmsnorm.wide_plan(1, 2048) == (512, 1)
    assert rmsnorm.wide_plan(1, 7680) == (512, 4)
    assert rmsnorm.wide_plan(2, 7936) == (256, 8)
    assert rmsnorm.wide_plan(4, 4096) == (128, 8)
    for rows, n in ((1, 256), (1, 504), (1, 8192), (2, 8192), (1, 7688), (1, 100)):
        assert rmsnorm.wide_plan(rows, n) is None, (rows, n)
    assert rmsnorm.gemv_norm_ok(1, 4096) and rmsnorm.gemv_norm_ok(2, 512)
    assert rmsnorm.gemv_norm_ok(2, 4096) and rmsnorm.gemv_norm_ok(1, 3072)
    # past four vectors per thread (k4 = 3 at 512 threads), more rows, odd n
    assert not rmsnorm.gemv_norm_ok(1, 4608) and not rmsnorm.gemv_norm_ok(1, 7680)
    assert not rmsnorm.gemv_norm_ok(3, 4096) and not rmsnorm.gemv_norm_ok(1, 4100)
