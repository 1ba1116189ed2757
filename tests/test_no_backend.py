"""Without the kernel library every fuser is a no-op (CPU).

The reference's fusers patch nothing and report False when their kernel
backend is absent (src/umic/integrate.py:653-655, 673-675), and its
gate_silu_mul falls back to eager (src/umic/kernels/fused_ffn.py:121-126).
Here ``UMIC_HIP_LIB`` points at a file that does not exist: ``apply()``
reports every kernel fusion as 0 / False, leaves every forward and the
transformers RoPE globals untouched, the hooks that are pure torch (the
in-place KV cache hook, the decode-graph runner) still install, and the
model's outputs are those of the unpatched model.  Direct wrapper calls
still raise UmicLibraryError.
"""

from __future__ import annotations

import pytest
import torch

from test_injection import _wrap, text_inputs, tiny_text_model, tiny_vision_model
from umic import _lib, integrate, optimize
from umic.kernels import fused_ffn

pytestmark = pytest.mark.filterwarnings("ignore::FutureWarning")


@pytest.fixture
def no_library(monkeypatch, tmp_path):
    monkeypatch.setenv("UMIC_HIP_LIB", str(tmp_path / "missing" / "libumic_hip.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "HAS_KERNELS", False)
    monkeypatch.setattr(_lib, "_load_error", None)
    yield
    integrate.unfuse_rope()


def test_apply_patches_nothing_without_the_library(no_library):
    from transformers.models.qwen3_vl import modeling_qwen3_vl as hf

    text_rope, vision_rope = hf.apply_rotary_pos_emb, hf.apply_rotary_pos_emb_vision
    lm = tiny_text_model()
    ref = tiny_text_model()
    model = _wrap(lm=lm, visual=tiny_vision_model(), expert=tiny_text_model(layers=1))
    report = optimize.apply(model)
    assert not _lib.available() and "missing" in _lib.load_error()
    kernel_keys = [k for k in report if k not in ("flow_cache_hook", "decode_graph")]
    assert kernel_keys and all(report[k] in (0, False) for k in kernel_keys), report
    assert report["flow_cache_hook"] is True and report["decode_graph"] is True
    # no instance forward anywhere below the LM, the ViT or the expert
    for scope in (model.vlm.language_model, model.vlm.visual, model.expert):
        assert not [n for n, m in scope.named_modules() if "forward" in m.__dict__]
    assert hf.apply_rotary_pos_emb is text_rope
    assert hf.apply_rotary_pos_emb_vision is vision_rope
    with torch.no_grad():
        out = lm(**text_inputs(lm)).last_hidden_state
        want = ref(**text_inputs(ref)).last_hidden_state
    assert torch.equal(out, want)
    # each fuser on its own reports the same
    assert integrate.fuse_mlps(lm) == 0 and integrate.fuse_linears(lm) == 0
    assert integrate.fuse_text_rope() is False and integrate.fuse_vision_rope() is False


def test_gate_silu_mul_falls_back_and_wrappers_raise(no_library):
    torch.manual_seed(0)
    x = torch.randn(8, 64).to(torch.bfloat16)
    wg, wu = (0.1 * torch.randn(64, 32)).to(torch.bfloat16), (0.1 * torch.randn(64, 32)).to(
        torch.bfloat16)
    assert torch.equal(fused_ffn.gate_silu_mul(x, wg, wu),
                       fused_ffn.gate_silu_mul_eager(x, wg, wu))
    with pytest.raises(_lib.UmicLibraryError):
        _lib.lib()
