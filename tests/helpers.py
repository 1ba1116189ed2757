"""Shared test helpers: bf16 bit views, ulp metrics, seeded inputs."""

from __future__ import annotations

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """uint16 bf16 bit patterns of a bf16 tensor (any device)."""
    assert t.dtype == torch.bfloat16, t.dtype
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16).copy()


def from_bits(a: np.ndarray, device="cpu") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def ulp(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """bf16 ulp distance of two uint16 bit arrays."""

    def ordered(v):
        v = np.asarray(v).astype(np.int32)
        return np.where((v & 0x8000) != 0, -(v & 0x7FFF), v & 0x7FFF)

    return np.abs(ordered(a) - ordered(b))


def ulp_hist(d: np.ndarray, cap: int = 4) -> dict:
    return {f"{i}": int((d == i).sum()) for i in range(cap)} | {f">={cap}": int((d >= cap).sum())}


def log_parity(op: str, shape, d: np.ndarray, against: str = "torch eager (GPU)") -> dict:
    """Record a bf16 ulp histogram of a kernel against eager: printed, and
    appended as a JSON line to the file named by $UMIC_PARITY_LOG if set."""
    import json
    import os

    rec = {"op": op, "shape": list(shape), "against": against, "elements": int(d.size),
           "max_ulp": int(d.max()) if d.size else 0, "hist": ulp_hist(d)}
    print(f"parity {op} {tuple(shape)} vs {against}: {rec['hist']}", flush=True)
    path = os.environ.get("UMIC_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    return rec


def bf16_randn(*shape, scale=1.0, shift=0.0, gen=None) -> torch.Tensor:
    """N(shift, scale^2) drawn on the CPU in fp32, then rounded to bf16."""
    return (shift + scale * torch.randn(*shape, generator=gen)).to(torch.bfloat16)


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """Norm-relative error, the reference's smoke-test metric
    (scripts/check_env.py:124-125)."""
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm())


def max_rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| / max |b| over the tensor."""
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).abs().max() / b.abs().max())


def qwen3_decoder_layer(device="cuda"):
    """BASELINE config 5 text decoder layer (hidden 4096, 32 q / 8 kv heads,
    head_dim 128, intermediate 12288; N(0, 0.02) weights, norms 1 + N(0, 0.1))
    in bf16 on `device`, and its rotary embedding."""
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import (Qwen3VLTextDecoderLayer,
                                                                Qwen3VLTextRotaryEmbedding)

    cfg = Qwen3VLTextConfig(hidden_size=4096, intermediate_size=12288, num_hidden_layers=1,
                            num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                            rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                            attn_implementation="sdpa")
    torch.manual_seed(0)
    layer = Qwen3VLTextDecoderLayer(cfg, 0)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.copy_(1 + 0.1 * torch.randn_like(p))
            else:
                p.copy_(0.02 * torch.randn_like(p))
    rot = Qwen3VLTextRotaryEmbedding(cfg)
    return layer.to(torch.bfloat16).to(device).eval(), rot.to(device)
