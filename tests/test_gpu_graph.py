"""GPU: the fused kernels inside a captured HIP graph (decode regime).

The reference replays its whole decode step from CUDA graphs
(src/umic/graph.py:155-167), so every fused kernel must be capture-safe: no
allocation by the library, no synchronisation, launches only on the given
stream.  Here a decode-shaped sequence of every entry point (M = 1 token, a
decoder layer's norms and RoPE, plus prefill-sized GEMMs so the MFMA kernels
are captured too) is captured once with torch.cuda.CUDAGraph, then replayed
several times on fresh inputs, with the program's own eager work and
synchronisations between replays; every replay must equal the eager result
bit for bit (same kernels, deterministic).  Nothing in the captured region
issues a memset.
"""

from __future__ import annotations

import pytest
import torch
from helpers import bf16_randn

from umic.kernels import fused_ffn, layernorm, linear, rmsnorm, rope

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed):
    g = torch.Generator().manual_seed(seed)
    return {
        "h": bf16_randn(1, 1, 4096, gen=g),
        "r": bf16_randn(1, 1, 4096, gen=g),
        "q": bf16_randn(1, 1, 32, 128, gen=g),
        "k": bf16_randn(1, 1, 8, 128, gen=g),
        "cos": bf16_randn(1, 1, 128, gen=g),
        "sin": bf16_randn(1, 1, 128, gen=g),
        "v": bf16_randn(64, 1280, gen=g),
        "vr": bf16_randn(64, 1280, gen=g),
        "x": bf16_randn(128, 512, gen=g),
        "xs": bf16_randn(300, 12288, gen=g),
        "hd": bf16_randn(1, 2, 512, gen=g),    # decode rows for the GEMVs
        "hr": bf16_randn(1, 2, 512, gen=g),
    }


def _step(t, p):
    """One decode-shaped pass over every fused entry point."""
    out = {}
    out["n1"] = rmsnorm.rmsnorm_hip(t["h"], p["w"], 1e-6)
    out["qn"] = rmsnorm.rmsnorm_hip(t["q"], p["wq"], 1e-6)
    out["kn"] = rmsnorm.rmsnorm_hip(t["k"], p["wq"], 1e-6)
    out["qr"], out["kr"] = rope.apply_rotary_text_hip(out["qn"].transpose(1, 2),
                                                      out["kn"].transpose(1, 2), t["cos"], t["sin"])
    out["n2"], out["s2"] = rmsnorm.add_rmsnorm_hip(t["h"], t["r"], p["w"], 1e-6)
    out["ln"] = layernorm.layernorm_hip(t["v"], p["lw"], p["lb"], 1e-6)
    out["aln"], out["as"] = layernorm.add_layernorm_hip(t["v"], t["vr"], p["lw"], p["lb"], 1e-6)
    out["lin"] = linear.linear_hip(t["x"], p["wl"])
    out["lin_sk"] = linear.linear_hip(t["xs"], p["wsk"])  # stream-K schedule
    out["p5"] = fused_ffn.gate_silu_mul_hip(t["x"], p["wg"].t(), p["wu"].t())
    # decode GEMVs: one linear, three in one launch, P5, down_proj + residual
    out["gv"] = linear.linear_hip(t["hd"], p["wl"])
    out["mq"], out["mk"], out["mv"] = linear.linear_multi_hip(
        t["hd"], [p["wl"], p["wg"], p["wu"]], [None, p["bg"], None])
    out["gp5"] = fused_ffn.gate_silu_mul_hip(t["hd"], p["wg"].t(), p["wu"].t())
    out["gadd"] = linear.linear_add_hip(out["gp5"], p["wd"], None, t["hr"])
    return out


def test_fused_kernels_replay_in_hip_graph():
    g = torch.Generator().manual_seed(99)
    p = {
        "w": bf16_randn(4096, scale=0.1, shift=1.0, gen=g).to(DEV),
        "wq": bf16_randn(128, scale=0.1, shift=1.0, gen=g).to(DEV),
        "lw": bf16_randn(1280, scale=0.1, shift=1.0, gen=g).to(DEV),
        "lb": bf16_randn(1280, scale=0.1, gen=g).to(DEV),
        "wl": bf16_randn(256, 512, scale=0.05, gen=g).to(DEV),
        "wg": bf16_randn(384, 512, scale=0.05, gen=g).to(DEV),
        "wu": bf16_randn(384, 512, scale=0.05, gen=g).to(DEV),
        "wsk": bf16_randn(264, 12288, scale=0.02, gen=g).to(DEV),
        "bg": bf16_randn(384, scale=0.1, gen=g).to(DEV),
        "wd": bf16_randn(512, 384, scale=0.05, gen=g).to(DEV),
    }
    from umic import _lib

    assert _lib.lib().umic_linear_workspace_bytes(300, 264, 12288) > 0
    static = {k: v.to(DEV) for k, v in _inputs(0).items()}
    # warm up on a side stream (as torch.cuda.graphs recommends), then capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _step(static, p)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _step(static, p)
    torch.cuda.synchronize()

    for seed in (1, 2, 3, 4):
        fresh = _inputs(seed)
        for k, v in fresh.items():
            static[k].copy_(v)
        graph.replay()
        # the program's own eager work between replays
        eager = _step({k: v.to(DEV) for k, v in fresh.items()}, p)
        torch.cuda.synchronize()
        for name, ref in eager.items():
            assert torch.equal(captured[name], ref), (seed, name)


def test_stream_k_workspace_outlives_a_captured_graph():
    """A graph captured with the stream-K linear keeps its workspace address.
    A later, larger eager call grows the per-stream workspace; the old buffer
    must stay allocated, so a tensor allocated afterwards is not overwritten
    when the graph replays, and the replay still computes the same product."""
    g = torch.Generator().manual_seed(7)
    xs = bf16_randn(300, 12288, gen=g).to(DEV)
    ws_ = bf16_randn(264, 12288, scale=0.02, gen=g).to(DEV)
    xb = bf16_randn(2816, 12288, gen=g).to(DEV)
    wb = bf16_randn(4096, 12288, scale=0.02, gen=g).to(DEV)
    assert linear.stream_k_planned(xs, ws_) and linear.stream_k_planned(xb, wb)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ref = linear.linear_hip(xs, ws_)          # allocates this stream's workspace
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            out = linear.linear_hip(xs, ws_)
        big = linear.linear_hip(xb, wb)           # grows the workspace
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    small_bytes = linear._lib.lib().umic_linear_workspace_bytes(300, 264, 12288)
    sentinel = torch.full((small_bytes,), 0x5A, dtype=torch.uint8, device=DEV)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert bool((sentinel == 0x5A).all())
    assert big.shape == (2816, 4096)


def test_four_wave_stream_k_replays_in_hip_graph():
    """The four-wave stream-K schedule (the down_proj path: K >= 8192 and
    most CUs' worth of tiles) captured in a HIP graph: its tile counters are
    left at zero by each launch, so replays on fresh inputs equal the eager
    call bit for bit, with eager launches on the same workspace between
    them."""
    g = torch.Generator().manual_seed(11)
    x = bf16_randn(3100, 8192, gen=g).to(DEV)
    w = bf16_randn(4096, 8192, scale=0.02, gen=g).to(DEV)
    assert linear.stream_k_planned(x, w)
    print("four-wave stream-K graph capture M=3100 N=4096 K=8192", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        linear.linear_hip(x, w)                   # this stream's workspace
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            out = linear.linear_hip(x, w)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for seed in range(3):
        gi = torch.Generator().manual_seed(100 + seed)
        x.copy_(bf16_randn(3100, 8192, gen=gi).to(DEV))
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            graph.replay()
            ref = linear.linear_hip(x, w)         # eager, same stream and workspace
        torch.cuda.synchronize()
        assert torch.equal(out, ref), seed
