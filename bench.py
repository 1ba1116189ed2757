"""UMIC hot-path benchmark on one MI355X (BASELINE.json metric and configs).

A step is one pass of the fused hot path over one batch of synthetic input at
the BASELINE shapes, every kernel launched once through the C ABI:

  rmsnorm          [3100, 4096]                     (config 2)
  add_rmsnorm      [3100, 4096]                     (config 2)
  layernorm        [16384, 1280] + bias             (config 2)
  add_layernorm    [16384, 1280] + bias             (config 2)
  rope_text        q [1,32,3100,128], k [1,8,3100,128], bf16 cos/sin (config 4)
  rope_vision      q, k [16384,16,80] views of packed qkv, fp32 cos/sin (config 4)
  q_proj, o_proj   [3100,4096] x [4096,4096]^T      (config 3)
  gate_silu_mul    [3100,4096] x 2 x [12288,4096]^T (config 3, P5)
  down_proj        [3100,12288] x [4096,12288]^T on this library's linear
                   (208 output tiles: the four-wave stream-K schedule),
                   which the fused MLP uses for this shape (the reference
                   keeps the vendor BLAS); with P5 it makes the LM MLP
                   prefill.
  down_proj_vendor the same GEMM on the vendor BLAS (F.linear, hipBLASLt),
                   measured beside it for that per-site choice.
  q_proj_vendor    q_proj on the vendor BLAS, which the fused path keeps
                   for q/o (this library's linear only ties it there).

Inputs are resident in HBM before timing.  Each HBM-bound kernel rotates
over its own ring of input sets (and keeps its outputs alive for one ring
turn) sized so a set is revisited only after >= 640 MB of other traffic:
nothing can be served from the 256 MB Infinity Cache.  Timing: the K launches
of one kernel run back-to-back between two HIP events recorded on the stream
they are launched on (torch's current stream); each group is preceded by an
untimed spacer launch (two P5 GEMMs) so the host has queued the whole group
before the first event fires and host launch latency never shows up as GPU
time.  ms_per_step is the sum over kernels of the per-launch event time.

Output: one JSON line (rank 0).  value = aggregate achieved HBM GB/s of the
six fused norm/RoPE kernels (algorithmic bytes / summed durations); each
HBM-bound kernel also carries the time of a plain device copy of its byte
count (copy_us, of_copy = copy time / kernel time) and of the library's tuned
streaming copy (umic_stream_copy: stream_copy_us, of_stream_copy), and
copy_ceiling_gbps / of_copy and stream_copy_ceiling_gbps / of_stream_copy
give the same for the six together;
mlp_prefill_ms = gate_silu_mul + down_proj; roofline = the dominant kernel
(by time) of the step, its traffic (HBM bytes per launch) measured at the
end of the run, after every timed step, by rocprofv3 --pmc child runs of --pmc-probe (FETCH_SIZE,
WRITE_SIZE, scaled by a device copy of known size; the committed PMC summary
when the profiler is absent or --no-traffic is given), and its clock_ghz from
a GRBM_GUI_ACTIVE pass of the same probe; cpu_baseline = the reference's own CPU path (HF's
eager Qwen3-VL modules, RoPE functions and the eager P5 chain in torch, bf16,
on the host cores) over all five BASELINE configs at full size, value in GB/s
over the norm/RoPE ops as for the GPU; cpu_oracle = the scalar C oracle (one
core) on a bounded quarter-row sample of the norm/RoPE workload.
layer = BASELINE config 5, one Qwen3-VL decoder layer eager vs fused at
prefill M=3100 and decode M=1 (plus the fused decode step replayed from a
HIP graph); decode_gemv = that decode step's four GEMV launches on weights
rotated past every cache (as in a many-layer decode), each beside a plain
streaming read of the same weight bytes (umic_stream_read; of_read = read
time / GEMV time); vit_encoder = BASELINE config 4 in context, the Qwen3-VL vision
encoder (4 blocks, 16384 tokens, hidden 1280) eager vs with the vision
fusions injected; --no-layer skips both.  kv_cache = text RoPE fused with the
in-place KV-cache append against RoPE + two slice copies, at prefill and at a
32-token flow step; --no-kv-cache skips it.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "umic-alpamayo_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
# the reference's norm / RoPE kernels, whose whole-job HBM throughput is `value`
VALUE_SITES = ("rmsnorm", "add_rmsnorm", "layernorm", "add_layernorm", "rope_text",
               "rope_vision")
BF16_PEAK_TFLOPS = 2500.0
METRIC = "fused-kernel HBM GB/s (% of peak) + LM MLP prefill ms at M=3100 bf16"


def _bf(*shape, scale=1.0, shift=0.0, gen=None):
    """N(shift, scale^2) bf16 tensor drawn directly on the GPU."""
    import torch

    return (shift + scale * torch.randn(*shape, generator=gen, device="cuda")).to(torch.bfloat16)


def build_workload():
    """Allocate every input on the GPU; return the list of kernel entries.

    Entry: (name, launch(step) -> None, algorithmic bytes, flops, bound).
    Algorithmic bytes count each tensor read or written exactly once
    (bf16 = 2 B, fp32 = 4 B); flops are 2*M*N*K per GEMM.
    """
    import torch

    from umic.kernels import fused_ffn, layernorm, linear, rmsnorm, rope

    g = torch.Generator(device="cuda").manual_seed(0)
    M, H = 3100, 4096
    MV, HV = 16384, 1280
    w_rms = _bf(H, scale=0.1, shift=1.0, gen=g)
    w_ln, b_ln = _bf(HV, scale=0.1, shift=1.0, gen=g), _bf(HV, scale=0.1, gen=g)

    # text RoPE tables (theta 1e6, positions 0..3099), bf16 as HF casts them
    D = 128
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.arange(M, dtype=torch.float32)[:, None] * inv[None]
    emb = torch.cat((ang, ang), -1)
    cos_t = emb.cos().to(torch.bfloat16)[None].cuda()
    sin_t = emb.sin().to(torch.bfloat16)[None].cuda()
    # vision RoPE tables: 16 images of 32x32 patches, merged h/w ids, theta 1e4
    hh, ww = torch.meshgrid(torch.arange(32), torch.arange(32), indexing="ij")
    blk = (16, 2, 16, 2)
    hp = hh.reshape(blk).transpose(1, 2).flatten()
    wp = ww.reshape(blk).transpose(1, 2).flatten()
    pid = torch.stack([hp, wp], -1).repeat(16, 1)
    vinv = 1.0 / (1e4 ** (torch.arange(0, 40, 2, dtype=torch.float32) / 40))
    vemb = (pid[..., None].float() * vinv).flatten(1)
    vemb = torch.cat((vemb, vemb), -1)
    cos_v, sin_v = vemb.cos().cuda(), vemb.sin().cuda()

    RING_BYTES = 640e6

    def ring(nbytes, make):
        n = max(2, min(16, int(-(-RING_BYTES // nbytes))))
        return [make() for _ in range(n)]

    rms_x = ring(4 * M * H, lambda: _bf(M, H, gen=g))
    add_xr = ring(8 * M * H, lambda: (_bf(M, H, gen=g), _bf(M, H, gen=g)))
    ln_x = ring(4 * MV * HV, lambda: _bf(MV, HV, gen=g))
    addln_xr = ring(8 * MV * HV, lambda: (_bf(MV, HV, gen=g), _bf(MV, HV, gen=g)))
    rope_qk = ring(4 * 40 * M * D, lambda: (_bf(1, M, 32, D, gen=g).transpose(1, 2),
                                            _bf(1, M, 8, D, gen=g).transpose(1, 2)))
    rope_qkv = ring(8 * 16 * MV * 80, lambda: _bf(MV, 3, 16, 80, gen=g))

    # GEMM operand sets rotate like the norm inputs: a set (x, weights, and
    # the output kept for one ring turn) comes back only after >= 640 MB
    FF = 12288
    proj = ring(2 * (2 * M * H + H * H), lambda: (_bf(M, H, gen=g), _bf(H, H, scale=0.02, gen=g),
                                                   _bf(H, H, scale=0.02, gen=g)))
    p5 = ring(2 * (M * H + 2 * FF * H + M * FF),
              lambda: (_bf(M, H, gen=g), _bf(FF, H, scale=0.02, gen=g),
                       _bf(FF, H, scale=0.02, gen=g)))
    down = ring(2 * (M * FF + H * FF + M * H),
                lambda: (_bf(M, FF, gen=g), _bf(H, FF, scale=0.02, gen=g)))
    qn_w, kn_w = _bf(D, scale=0.1, shift=1.0, gen=g), _bf(D, scale=0.1, shift=1.0, gen=g)
    eps = 1e-6

    def pick(r, i):
        return r[i % len(r)]

    def unfused_qk_norm_rope(q, k):
        qn = rmsnorm.rmsnorm_hip(q.transpose(1, 2), qn_w, eps).transpose(1, 2)
        kn = rmsnorm.rmsnorm_hip(k.transpose(1, 2), kn_w, eps).transpose(1, 2)
        return rope.apply_rotary_text_hip(qn, kn, cos_t, sin_t)

    def vision(i):
        q, k, _ = pick(rope_qkv, i).permute(1, 0, 2, 3).unbind(0)
        return rope.apply_rotary_vision_hip(q, k, cos_v, sin_v)

    b2 = 2
    ents = [
        ("rmsnorm", lambda i: rmsnorm.rmsnorm_hip(pick(rms_x, i), w_rms, eps),
         2 * M * H * b2 + H * b2, 0, "hbm"),
        ("add_rmsnorm", lambda i: rmsnorm.add_rmsnorm_hip(*pick(add_xr, i), w_rms, eps),
         4 * M * H * b2 + H * b2, 0, "hbm"),
        ("layernorm", lambda i: layernorm.layernorm_hip(pick(ln_x, i), w_ln, b_ln, eps),
         2 * MV * HV * b2 + 2 * HV * b2, 0, "hbm"),
        ("add_layernorm", lambda i: layernorm.add_layernorm_hip(*pick(addln_xr, i), w_ln, b_ln,
                                                                eps),
         4 * MV * HV * b2 + 2 * HV * b2, 0, "hbm"),
        ("rope_text", lambda i: rope.apply_rotary_text_hip(*pick(rope_qk, i), cos_t, sin_t),
         2 * b2 * (32 + 8) * M * D + 2 * b2 * M * D, 0, "hbm"),
        ("rope_vision", vision, 2 * b2 * 2 * 16 * MV * 80 + 2 * 4 * MV * 80, 0, "hbm"),
        # the attention's q_norm / k_norm fused into the text RoPE (not one of
        # the reference's kernels: reported, not part of `value`)
        ("qk_norm_rope", lambda i: rope.qk_norm_rope(*pick(rope_qk, i), cos_t, sin_t, qn_w, kn_w,
                                                     eps),
         2 * b2 * (32 + 8) * M * D + 2 * b2 * M * D + 2 * b2 * D, 0, "hbm"),
        # the same work unfused: the two head-row norms, then the RoPE
        ("qk_norm_rope_unfused", lambda i: unfused_qk_norm_rope(*pick(rope_qk, i)),
         2 * b2 * (32 + 8) * M * D + 2 * b2 * M * D + 2 * b2 * D, 0, "hbm"),
        ("q_proj", lambda i: linear.linear_hip(pick(proj, i)[0], pick(proj, i)[1]),
         (M * H + H * H + M * H) * b2, 2 * M * H * H, "mfma"),
        ("o_proj", lambda i: linear.linear_hip(pick(proj, i)[0], pick(proj, i)[2]),
         (M * H + H * H + M * H) * b2, 2 * M * H * H, "mfma"),
        ("gate_silu_mul", lambda i: fused_ffn.gate_silu_mul_hip(pick(p5, i)[0], pick(p5, i)[1].t(),
                                                                pick(p5, i)[2].t()),
         (M * H + 2 * FF * H + M * FF) * b2, 2 * 2 * M * FF * H, "mfma"),
        ("down_proj", lambda i: linear.linear_hip(*pick(down, i)),
         (M * FF + H * FF + M * H) * b2, 2 * M * H * FF, "mfma"),
        # the q/o projection on the vendor BLAS, which the fused path keeps for it
        ("q_proj_vendor", lambda i: torch.nn.functional.linear(pick(proj, i)[0], pick(proj, i)[1]),
         (M * H + H * H + M * H) * b2, 2 * M * H * H, "mfma"),
        ("down_proj_vendor", lambda i: torch.nn.functional.linear(*pick(down, i)),
         (M * FF + H * FF + M * H) * b2, 2 * M * H * FF, "mfma"),
    ]
    rings = {"rmsnorm": len(rms_x), "add_rmsnorm": len(add_xr), "layernorm": len(ln_x),
             "add_layernorm": len(addln_xr), "rope_text": len(rope_qk),
             "rope_vision": len(rope_qkv), "qk_norm_rope": len(rope_qk),
             "qk_norm_rope_unfused": len(rope_qk), "q_proj": len(proj), "o_proj": len(proj),
             "gate_silu_mul": len(p5), "down_proj": len(down), "q_proj_vendor": len(proj),
             "down_proj_vendor": len(down)}
    spacer = lambda: fused_ffn.gate_silu_mul_hip(p5[0][0], p5[0][1].t(), p5[0][2].t())  # noqa: E731
    return ents, rings, spacer


def cpu_oracle(sample_s: float) -> dict:
    """Time the CPU oracle (scalar C, one core) on a bounded sample of the
    norm/RoPE workload: the restatement the parity tests check against,
    reported beside the reference's own CPU path."""
    import numpy as np

    import oracle

    oracle._load()
    rng = np.random.default_rng(0)

    def bfr(*shape, scale=1.0, shift=0.0):
        return oracle.bf16_from_f32((shift + scale * rng.standard_normal(shape)).astype(
            np.float32))

    # Row subsets of the GPU shapes (1/4 of the rows), repeated until the
    # sample time is spent; bytes are counted as for the GPU kernels.
    M, H, MV, HV, D = 3100 // 4, 4096, 16384 // 4, 1280, 128
    x, r, w = bfr(M, H), bfr(M, H), bfr(H, scale=0.1, shift=1.0)
    xv, rv = bfr(MV, HV), bfr(MV, HV)
    wl, bl = bfr(HV, scale=0.1, shift=1.0), bfr(HV, scale=0.1)
    q, k = bfr(M, 32, D), bfr(M, 8, D)
    ct, st = bfr(M, D), bfr(M, D)
    vq, vk = bfr(MV, 16, 80), bfr(MV, 16, 80)
    cv = rng.standard_normal((MV, 80)).astype(np.float32)
    sv = rng.standard_normal((MV, 80)).astype(np.float32)
    work = [
        (lambda: oracle.rmsnorm(x, w, 1e-6), 4 * M * H),
        (lambda: oracle.add_rmsnorm(x, r, w, 1e-6), 8 * M * H),
        (lambda: oracle.layernorm(xv, wl, bl, 1e-6), 4 * MV * HV),
        (lambda: oracle.add_layernorm(xv, rv, wl, bl, 1e-6), 8 * MV * HV),
        (lambda: (oracle.rope_text(q, ct, st), oracle.rope_text(k, ct, st)),
         4 * 40 * M * D + 4 * M * D),
        (lambda: (oracle.rope_vision(vq, cv, sv), oracle.rope_vision(vk, cv, sv)),
         4 * 32 * MV * 80 + 8 * MV * 80),
    ]
    tot_b, tot_t, passes = 0, 0.0, 0
    t_end = time.perf_counter() + sample_s
    while time.perf_counter() < t_end or passes == 0:
        for fn, nbytes in work:
            t0 = time.perf_counter()
            fn()
            tot_t += time.perf_counter() - t0
            tot_b += nbytes
        passes += 1
    return {"value": round(tot_b / tot_t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{passes} pass(es) of the six norm/RoPE oracle functions on 1/4 of the "
                      f"BASELINE rows ({tot_b / passes / 1e6:.0f} MB per pass), "
                      f"{tot_t:.1f} s of single-thread scalar C"}


def _host_cpu() -> dict:
    """CPU model, the bf16 matrix/vector features torch's CPU kernels use,
    and the cores this process may run on."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    feats = {k: k in flags for k in ("amx_bf16", "amx_tile", "avx512_bf16", "avx512f")}
    return {"cpu_model": model, "cpu_flags": feats, "affinity_cpus": len(os.sched_getaffinity(0))}


def cpu_reference(budget_s: float) -> dict:
    """The reference's eager CPU path over the BASELINE configs, on the host.

    The reference falls back to eager torch wherever a kernel is unavailable
    (src/umic/kernels/fused_ffn.py:31-43 for P5; the modules' own forwards
    for the norms, linears and RoPE), so its CPU path is HF transformers'
    Qwen3-VL modules and functions run by torch in bf16:

      config 1  RMSNorm [256,1024] -> HF MLP 1024->3072->1024 (silu)
      config 2  RMSNorm, residual add + RMSNorm [3100,4096];
                LayerNorm, residual add + LayerNorm [16384,1280]
      config 3  gate_silu_mul_eager [3100,4096] x [4096,12288] x 2, down_proj
                F.linear 12288->4096, q_proj / o_proj F.linear 4096->4096
      config 4  apply_rotary_pos_emb q [1,32,3100,128] k [1,8,3100,128];
                apply_rotary_pos_emb_vision q, k [16384,16,80], fp32 tables
      config 5  one Qwen3-VL text decoder layer, prefill M=3100, then one
                decode step (M=1) on the prefill's KV cache

    Full BASELINE sizes.  Inputs are drawn in fp32 with a fixed seed and cast
    to bf16.  Each op: 2 warm-up calls, then the median of 5 (1 and 3 for the
    M=3100 GEMMs and the layer); an op whose first call shows the budget
    would be exceeded gets fewer repetitions (at least one timed call).
    Threads: every CPU of this process's affinity mask, capped by
    OMP_NUM_THREADS when the environment sets it (the host share of a
    one-GPU box).  value = the norm/RoPE ops' bytes (counted as for the GPU
    kernels) over their summed medians, in GB/s, as the GPU's value."""
    import torch
    from torch.nn import functional as F
    from transformers.models.qwen3_vl import modeling_qwen3_vl as hf
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig

    host = _host_cpu()
    threads = host["affinity_cpus"]
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, max(1, int(os.environ["OMP_NUM_THREADS"])))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)
    bf = torch.bfloat16

    def bfr(*shape, scale=1.0, shift=0.0):
        return (shift + scale * torch.randn(*shape, generator=gen)).to(bf)

    t_budget = time.perf_counter() + budget_s
    ms: dict[str, float] = {}
    reps_used: dict[str, int] = {}

    def timed(name, fn, warm=2, reps=5):
        t0 = time.perf_counter()
        fn()
        first = time.perf_counter() - t0  # the first warm-up call
        fit = int((t_budget - time.perf_counter()) / max(first, 1e-6))  # calls that fit
        reps = max(1, min(reps, fit))
        warm = max(0, min(warm - 1, fit - reps))
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        ts.sort()
        ms[name] = round(ts[len(ts) // 2] * 1e3, 3)
        reps_used[name] = reps

    def text_cfg(hidden, inter, heads=32, kv=8, hd=128):
        return Qwen3VLTextConfig(hidden_size=hidden, intermediate_size=inter,
                                 num_attention_heads=heads, num_key_value_heads=kv,
                                 head_dim=hd, num_hidden_layers=1, rms_norm_eps=1e-6,
                                 hidden_act="silu",
                                 rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                                 attn_implementation="sdpa")

    def init_(mod):
        with torch.no_grad():
            for n, p in mod.named_parameters():
                if "norm" in n:
                    p.copy_(1 + 0.1 * torch.randn(p.shape, generator=gen))
                else:
                    p.copy_(0.02 * torch.randn(p.shape, generator=gen))
        return mod.to(bf).eval()

    M, H, MV, HV, D = 3100, 4096, 16384, 1280, 128
    nbytes = {}
    with torch.no_grad():
        # config 1: the CPU-eager MLP block
        c1 = text_cfg(1024, 3072, heads=8, kv=8, hd=128)
        norm1, mlp1 = init_(hf.Qwen3VLTextRMSNorm(1024, eps=1e-6)), init_(hf.Qwen3VLTextMLP(c1))
        x1 = bfr(256, 1024)
        timed("c1_mlp_block", lambda: mlp1(norm1(x1)))

        # config 2: the norms at full size
        x, r = bfr(M, H), bfr(M, H)
        rms = init_(hf.Qwen3VLTextRMSNorm(H, eps=1e-6))
        xv, rv = bfr(MV, HV), bfr(MV, HV)
        ln = torch.nn.LayerNorm(HV, eps=1e-6)
        with torch.no_grad():
            ln.weight.copy_(bfr(HV, scale=0.1, shift=1.0).float())
            ln.bias.copy_(bfr(HV, scale=0.1).float())
        ln = ln.to(bf)
        timed("rmsnorm", lambda: rms(x))
        timed("add_rmsnorm", lambda: rms(x + r))
        timed("layernorm", lambda: ln(xv))
        timed("add_layernorm", lambda: ln(xv + rv))
        nbytes.update(rmsnorm=4 * M * H + 2 * H, add_rmsnorm=8 * M * H + 2 * H,
                      layernorm=4 * MV * HV + 4 * HV, add_layernorm=8 * MV * HV + 4 * HV)
        del x, r, xv, rv

        # config 4: RoPE at full size (q/k as transposed projection views)
        q, k = bfr(1, M, 32, D).transpose(1, 2), bfr(1, M, 8, D).transpose(1, 2)
        inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        emb = torch.arange(M, dtype=torch.float32)[:, None] * inv[None]
        emb = torch.cat((emb, emb), -1)
        ct, st = emb.cos().to(bf)[None], emb.sin().to(bf)[None]
        vq, vk = bfr(MV, 16, 80), bfr(MV, 16, 80)
        cv, sv = torch.randn(MV, 80, generator=gen), torch.randn(MV, 80, generator=gen)
        timed("rope_text", lambda: hf.apply_rotary_pos_emb(q, k, ct, st))
        timed("rope_vision", lambda: hf.apply_rotary_pos_emb_vision(vq, vk, cv, sv))
        nbytes.update(rope_text=4 * 40 * M * D + 4 * M * D,
                      rope_vision=4 * 32 * MV * 80 + 8 * MV * 80)
        del q, k, vq, vk

        # config 3: the M=3100 projections, W ~ N(0, 0.02)
        xg = bfr(M, H)
        wg, wu = bfr(12288, H, scale=0.02), bfr(12288, H, scale=0.02)
        wd, wq, wo = bfr(H, 12288, scale=0.02), bfr(H, H, scale=0.02), bfr(H, H, scale=0.02)
        ffn_eager = lambda a, g_, u_: F.silu(a @ g_) * (a @ u_)  # noqa: E731  fused_ffn.py:43
        hmid = ffn_eager(xg, wg.t(), wu.t())
        timed("gate_silu_mul", lambda: ffn_eager(xg, wg.t(), wu.t()), warm=1, reps=3)
        timed("down_proj", lambda: F.linear(hmid, wd), warm=1, reps=3)
        timed("q_proj", lambda: F.linear(xg, wq), warm=1, reps=3)
        timed("o_proj", lambda: F.linear(xg, wo), warm=1, reps=3)
        del xg, wg, wu, wd, wq, wo, hmid

        # config 5: one decoder layer, prefill then one decode step
        c5 = text_cfg(H, 12288)
        layer = init_(hf.Qwen3VLTextDecoderLayer(c5, 0))
        rot = hf.Qwen3VLTextRotaryEmbedding(c5)
        h0 = bfr(1, M, H)
        pos = torch.arange(M)[None]
        cs = rot(h0, pos)
        from transformers.cache_utils import DynamicCache

        def prefill():
            cache = DynamicCache()
            layer(h0, position_embeddings=cs, past_key_values=cache, position_ids=pos)
            return cache

        timed("layer_prefill", prefill, warm=1, reps=3)
        cache = prefill()
        h1 = bfr(1, 1, H)
        cs1 = rot(h1, torch.tensor([[M]]))

        def decode():
            layer(h1, position_embeddings=cs1, past_key_values=cache,
                  position_ids=torch.tensor([[M]]))
            cache.crop(-1)

        timed("layer_decode", decode)

    sites = list(nbytes)
    tot_ms = sum(ms[n] for n in sites)
    value = sum(nbytes.values()) / (tot_ms * 1e-3) / 1e9
    flops = {"gate_silu_mul": 4 * M * 12288 * H, "down_proj": 2 * M * H * 12288,
             "q_proj": 2 * M * H * H, "o_proj": 2 * M * H * H}
    return {"value": round(value, 3), "unit": "GB/s", "cores": threads, "kind": "reference",
            "mlp_prefill_ms": round(ms["gate_silu_mul"] + ms["down_proj"], 3),
            "ms": ms, "reps": reps_used,
            "gemm_tflops": {n: round(f / (ms[n] * 1e-3) / 1e12, 3) for n, f in flops.items()},
            **host,
            "sample": "the reference's eager CPU path (HF transformers Qwen3-VL modules and "
                      "RoPE functions, fused_ffn.py:31-43's gate_silu_mul_eager, F.linear) "
                      "on all five BASELINE configs at full size, bf16, torch on "
                      f"{threads} threads; value over the six norm/RoPE ops "
                      f"({sum(nbytes.values()) / 1e6:.0f} MB in {tot_ms:.1f} ms)"}


def load_traffic(name: str):
    """Measured HBM bytes per launch from the committed rocprofv3 PMC summary
    (profiles/traffic_<kernel>.json), or None if none was committed."""
    p = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("hbm_bytes_per_launch")


# kernel-name fragment of each bench entry whose traffic can be measured live
# (a probe launches one entry only, so q/o and down_proj may share a kernel)
TRAFFIC_KERNELS = {"gate_silu_mul": "gemm_w4_kernel<2,", "q_proj/o_proj": "gemm_w4_kernel<1,",
                   "down_proj": "gemm_w4_kernel<1,"}
COPY_KERNEL = "__amd_rocclr_copyBuffer"  # the HIP runtime's device copy (the probe's calibration)


def measure_traffic(name: str):
    """HBM bytes per launch of bench entry `name`, measured in this run.

    Child runs of ``rocprofv3 --pmc FETCH_SIZE`` (then ``WRITE_SIZE``) over
    this script's ``--pmc-probe`` mode, restricted to the calibration copy and
    that kernel (one launch each, after a 1 GiB fill that evicts the Infinity
    Cache).  Each counter is scaled by what it reads for the copy, which moves
    exactly COPY_BYTES each way.  A third pass reads GRBM_GUI_ACTIVE, the GPU
    clock cycles the launch kept the graphics engine busy (summed over the
    XCDs), from which the caller derives the clock the kernel ran at.
    Returns (bytes, counters, None) or (None, None, reason) when the profiler
    is absent or a pass fails.
    """
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile

    frag = TRAFFIC_KERNELS.get(name)
    prof = shutil.which("rocprofv3")
    if frag is None or prof is None:
        return None, None, "no live measurement for this kernel" if prof else "rocprofv3 not found"
    env = dict(os.environ, TMPDIR="/tmp")
    vals = {}
    with tempfile.TemporaryDirectory(prefix="umic_pmc_", dir="/tmp") as tmp:
        for counter in ("FETCH_SIZE", "WRITE_SIZE", "GRBM_GUI_ACTIVE"):
            out = os.path.join(tmp, counter)
            # a pass takes a few seconds; the kill bound keeps a stuck profiler
            # from holding the run
            cmd = ["timeout", "-s", "KILL", "90", prof, "--pmc", counter, "-d", out, "-o",
                   "probe", "--output-format", "csv", "--", sys.executable, "-u",
                   os.path.abspath(__file__), "--pmc-probe", "--probe-only", name]
            r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
            if r.returncode != 0:
                return None, None, f"{counter} pass exited with {r.returncode}"
            files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
            if not files:
                return None, None, f"{counter} pass wrote no counter file"
            with open(files[0]) as f:
                vals[counter] = pmc_copy_and_kernel(csv.DictReader(f), frag)
            if vals[counter] is None:
                return None, None, f"{counter} pass: calibration copy or kernel not found"
    nbytes, info = calibrated_traffic(vals["FETCH_SIZE"], vals["WRITE_SIZE"])
    info["grbm_gui_active"] = vals["GRBM_GUI_ACTIVE"][1]
    return nbytes, info, None


def pmc_copy_and_kernel(rows, frag: str):
    """(calibration copy's counter value, kernel's value) from rocprofv3
    counter-collection rows (one row per dispatch), the last dispatch of
    each; None if either is missing or the copy read zero."""
    copy, kern = [], []
    for r in rows:
        if COPY_KERNEL in r["Kernel_Name"]:
            copy.append(float(r["Counter_Value"]))
        elif frag in r["Kernel_Name"]:
            kern.append(float(r["Counter_Value"]))
    if not copy or not kern or copy[-1] <= 0:
        return None
    return copy[-1], kern[-1]


def calibrated_traffic(fetch, write):
    """HBM bytes of the kernel from (copy KB, kernel KB) of FETCH_SIZE and of
    WRITE_SIZE: each counter scaled by COPY_BYTES over what it read for the
    copy, which moves exactly COPY_BYTES each way."""
    true_kb = COPY_BYTES / 1024
    rs, ws = true_kb / fetch[0], true_kb / write[0]
    nbytes = (fetch[1] * rs + write[1] * ws) * 1024
    return int(nbytes), {"fetch_kb": fetch[1], "write_kb": write[1],
                         "read_scale": round(rs, 4), "write_scale": round(ws, 4)}


def pmc_probe(only=None) -> int:
    """One launch of each kernel (or of the entries named in ``only``) after a
    plain device copy of known size.

    Run under ``rocprofv3 --pmc FETCH_SIZE`` (then ``WRITE_SIZE``): the copy
    reads and writes exactly COPY_BYTES, which calibrates the counters'
    per-dispatch byte figures for the kernels that follow.
    """
    import torch

    from umic import _lib

    _lib.load()
    torch.cuda.set_device(0)
    from umic.kernels import rope

    ents, _, _ = build_workload()
    src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda").normal_()
    dst = torch.empty_like(src)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    # text RoPE + KV append at the prefill shape (kv_cache_step's first case)
    S, D = 3100, 128
    q, k, v = (_bf(1, S, H, D).transpose(1, 2) for H in (32, 8, 8))
    kc, vc = (torch.empty(1, 8, 3200, D, dtype=torch.bfloat16, device="cuda") for _ in range(2))
    cs = torch.randn(1, S, D, device="cuda").to(torch.bfloat16)
    kv = ("rope_kv_append", lambda i: rope.rope_kv_append(q, k, v, cs, cs, kc, vc, 0),
          2 * 2 * 48 * S * D + 2 * 2 * S * D)
    torch.cuda.synchronize()
    # one kernel per probe: the unfused comparison (three launches) is left out
    single = [e for e in ents if not e[0].endswith("_unfused")] + [kv]
    if only:
        single = [e for e in single if e[0] in only]
    for name, fn, nbytes, *_ in [("copy", lambda i: dst.copy_(src), 2 * COPY_BYTES)] + single:
        flush.zero_()  # evict the Infinity Cache between probes
        torch.cuda.synchronize()
        fn(0)
        torch.cuda.synchronize()
        print(f"probe {name} algorithmic_bytes={nbytes}", flush=True)
    return 0


COPY_BYTES = 512 << 20


def copy_ceiling() -> int:
    """Practical HBM ceiling at the norm/RoPE sizes: torch's own device copy
    (read n, write n) of the same byte counts, back-to-back over 12 buffers,
    then the library's streaming copy (umic_stream_copy) over the same
    buffers; each timed group queued behind two spacer GEMMs so the host's
    launch cost stays out of the events."""
    import torch

    from umic import _lib

    torch.cuda.set_device(0)
    _lib.load()
    sa = torch.randn(8192, 8192, device="cuda").to(torch.bfloat16)

    def timed(fn, nbuf):
        for i in range(nbuf):
            fn(i)
        torch.cuda.synchronize()
        sa @ sa
        sa @ sa
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(nbuf):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / nbuf * 1e3

    for moved in (50_798_592, 83_891_200, 101_588_992, 167_777_280, 178_257_920,
                  400_000_000, 2 << 30):
        n = moved // 4  # bf16 elements per side
        nbuf = 12 if moved < (1 << 30) else 3
        src = [torch.empty(n, dtype=torch.bfloat16, device="cuda").normal_() for _ in range(nbuf)]
        dst = [torch.empty_like(src[0]) for _ in range(nbuf)]
        st = _lib.stream_of(src[0])
        us = timed(lambda i: dst[i].copy_(src[i]), nbuf)
        sus = timed(lambda i: _lib.call("umic_stream_copy", src[i].data_ptr(), dst[i].data_ptr(),
                                        moved // 2, st), nbuf)
        print(json.dumps({"copy_bytes_moved": moved, "us": round(us, 2),
                          "gbps": round(moved / us / 1e3, 1), "stream_copy_us": round(sus, 2),
                          "stream_copy_gbps": round(moved / sus / 1e3, 1)}), flush=True)
        del src, dst
    return 0


def same_bytes_copy(moved: int, steps: int, spacer=None) -> float:
    """Event-timed microseconds of one device copy (torch copy_, the HIP
    runtime's blit kernel) that reads moved/2 and writes moved/2 bytes: the
    practical ceiling of an HBM-bound kernel moving the same bytes.  The
    pairs rotate like the kernels' input rings (a pair returns only after
    >= 640 MB of other traffic), so the Infinity Cache serves none of it."""
    import torch

    n = moved // 4  # bf16 elements per side
    pairs = max(2, min(16, int(-(-640e6 // moved))))
    src = [torch.empty(n, dtype=torch.bfloat16, device="cuda").normal_() for _ in range(pairs)]
    dst = [torch.empty_like(src[0]) for _ in range(pairs)]
    for i in range(pairs):
        dst[i].copy_(src[i])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if spacer is not None:  # queued ahead, as before the kernels' groups
        spacer()
        spacer()
    e0.record()
    for i in range(steps):
        dst[i % pairs].copy_(src[i % pairs])
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps * 1e3


def stream_copy_us(moved: int, steps: int, spacer=None) -> float:
    """Event-timed microseconds of the library's streaming copy
    (umic_stream_copy: one-shot grid, non-temporal 16-byte loads and stores)
    reading moved/2 and writing moved/2 bytes, over rotating pairs as in
    same_bytes_copy: the tuned ceiling of a read-once / write-once kernel
    moving the same bytes (the runtime's blit copy is the plain one)."""
    import torch

    from umic import _lib

    side = moved // 2 // 16 * 16
    pairs = max(2, min(16, int(-(-640e6 // moved))))
    src = [torch.empty(side, dtype=torch.uint8, device="cuda").random_(0, 255)
           for _ in range(pairs)]
    dst = [torch.empty_like(src[0]) for _ in range(pairs)]
    st = _lib.stream_of(src[0])

    def copy(i):
        _lib.call("umic_stream_copy", src[i % pairs].data_ptr(), dst[i % pairs].data_ptr(),
                  side, st)

    for i in range(pairs):
        copy(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if spacer is not None:
        spacer()
        spacer()
    e0.record()
    for i in range(steps):
        copy(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps * 1e3


def _ring_len(nbytes: int) -> int:
    """Copies of an nbytes operand set so that a set returns only after
    >= 640 MB of other reads: the 256 MB Infinity Cache serves none of it."""
    return max(2, min(24, int(-(-640e6 // nbytes))))


def _graph_us(fn, n: int, reps: int) -> float:
    """Microseconds per launch of fn(i), i cycling over n ring slots, from a
    HIP graph of `reps` such launches (as a decode step replays them: the
    host's per-call cost, which exceeds these kernels' run time, stays out),
    replayed three times between two events."""
    import torch

    for i in range(n):
        fn(i)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(reps):
            fn(i % n)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / (3 * reps) * 1e3
    del graph
    return us


def stream_read_us(nbytes: int, reps: int) -> float:
    """Microseconds of one plain streaming read of nbytes (umic_stream_read),
    graph-replayed over a ring of buffers that no cache holds: the practical
    ceiling of a kernel that reads those bytes once."""
    import torch

    from umic import _lib

    nbytes = nbytes // 16 * 16
    n = _ring_len(nbytes)
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 255)
            for _ in range(n)]
    fold = torch.empty(_lib.UMIC_STREAM_READ_GRID, dtype=torch.int32, device="cuda")
    return _graph_us(lambda i: _lib.call("umic_stream_read", bufs[i].data_ptr(), nbytes,
                                         fold.data_ptr(), _lib.stream_of(fold)), n, reps)


def decode_gemv_step(reps: int = 60) -> dict:
    """The BASELINE config-5 decode step's four weight streams (one row, the
    library's GEMV launches exactly as the fused layer issues them) on
    weights rotated so that no cache holds them -- as in a decode over a
    many-layer model -- each beside umic_stream_read over the same weight
    bytes: of_read = read time / GEMV time (1.0 = as fast as reading the
    weights once)."""
    import torch

    from umic.kernels import fused_ffn, linear

    H, KV, FF, eps = 4096, 1024, 12288, 1e-6
    gen = torch.Generator(device="cuda").manual_seed(0)
    x, r = _bf(1, H, gen=gen), _bf(1, H, gen=gen)
    nw = _bf(H, scale=0.1, shift=1.0, gen=gen)
    h = _bf(1, FF, gen=gen)

    def site(shapes, launch):
        nbytes = sum(2 * a * b for a, b in shapes)
        n = _ring_len(nbytes)
        ws = [[_bf(a, b, scale=0.02, gen=gen) for a, b in shapes] for _ in range(n)]
        us = _graph_us(lambda i: launch(ws[i]), n, reps)
        del ws
        torch.cuda.empty_cache()
        read = stream_read_us(nbytes, reps)
        torch.cuda.empty_cache()
        return {"us": round(us, 2), "read_us": round(read, 2), "of_read": round(read / us, 3),
                "weight_mb": round(nbytes / 1e6, 1), "gbps": round(nbytes / us / 1e3, 1)}

    res = {
        "qkv_norm": site([(H, H), (KV, H), (KV, H)],
                         lambda w: linear.rmsnorm_linear_multi_hip(x, nw, eps, w)),
        "o_proj": site([(H, H)], lambda w: linear.linear_hip(x, w[0])),
        "add_norm_gate_silu_mul": site(
            [(FF, H), (FF, H)],
            lambda w: fused_ffn.add_rmsnorm_gate_silu_mul_hip(x, r, nw, eps, w[0].t(), w[1].t())),
        "down_proj_add": site([(H, FF)], lambda w: linear.linear_add_hip(h, w[0], None, x)),
    }
    sites = list(res.values())
    res["sum_us"] = round(sum(v["us"] for v in sites), 2)
    res["read_sum_us"] = round(sum(v["read_us"] for v in sites), 2)
    return res


def _config5_layer():
    """BASELINE config 5 text decoder layer in bf16 on the GPU with random
    N(0, 0.02) weights (norms 1 + N(0, 0.1)), its rotary embedding and the
    generator that drew them."""
    import torch
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import (Qwen3VLTextDecoderLayer,
                                                                Qwen3VLTextRotaryEmbedding)

    cfg = Qwen3VLTextConfig(hidden_size=4096, intermediate_size=12288, num_hidden_layers=1,
                            num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                            rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                            attn_implementation="sdpa")
    gen = torch.Generator(device="cuda").manual_seed(0)
    layer = Qwen3VLTextDecoderLayer(cfg, 0).to(torch.bfloat16).to("cuda").eval()
    with torch.no_grad():
        for name, prm in layer.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                prm.copy_(1 + 0.1 * torch.randn(prm.shape, generator=gen, device="cuda"))
            else:
                prm.copy_(0.02 * torch.randn(prm.shape, generator=gen, device="cuda"))
    rot = Qwen3VLTextRotaryEmbedding(cfg).to("cuda")
    return layer, rot, gen


def decode_layer() -> int:
    """Ten fused decode steps (one row) of the config-5 layer, every fuse_*
    of apply() injected, for a kernel trace of the decode step
    (``rocprofv3 --kernel-trace --stats -- python bench.py --decode-layer``):
    the GEMM sites run on the library's GEMV, norms and RoPE fused."""
    import torch

    from umic import _lib, integrate

    _lib.load()
    torch.cuda.set_device(0)
    layer, rot, gen = _config5_layer()
    h = _bf(1, 1, 4096, gen=gen)
    cs = rot(h, torch.arange(1, device="cuda")[None])
    with torch.no_grad():
        integrate.fuse_mlps(layer)
        integrate.fuse_linears(layer)
        integrate.fuse_rmsnorms(layer)
        integrate.fuse_add_rmsnorm(layer)
        integrate.fuse_text_rope()
        integrate.fuse_kv_rope(layer)
        for i in range(13):
            layer(h, position_embeddings=cs)
            torch.cuda.synchronize()
            if i >= 3:
                print(f"decode step {i - 3} done", flush=True)
    return 0


def layer_step() -> dict:
    """one Qwen3-VL text decoder layer (hidden 4096, 32 q /
    8 kv heads, head_dim 128, intermediate 12288, random N(0, 0.02) weights,
    norms 1 + N(0, 0.1)) timed eager and with the fused path injected
    (fuse_mlps, fuse_linears, fuse_rmsnorms, fuse_add_rmsnorm, fuse_text_rope,
    fuse_kv_rope -- with no cache, q_norm / k_norm / RoPE in one launch):
    prefill at M=3100 (also with the reference's q/o rule, the tiled linear
    from 64 rows: prefill_M3100_umic_tiled_qo_ms) and decode at M=1, the
    decode step also captured in a HIP graph (torch.cuda.CUDAGraph) and
    replayed, as the reference's decode runner does
    (src/umic/graph.py:155-167)."""
    import torch

    from umic import integrate

    layer, rot, gen = _config5_layer()
    inputs = {}
    for M in (3100, 1):
        h = _bf(1, M, 4096, gen=gen)
        inputs[M] = (h, rot(h, torch.arange(M, device="cuda")[None]))

    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3  # us

    res = {}
    with torch.no_grad():
        run = {M: (lambda h=h, cs=cs: layer(h, position_embeddings=cs))
               for M, (h, cs) in inputs.items()}
        for _ in range(10):
            run[3100]()
        res["prefill_M3100_eager_ms"] = round(
            statistics.median(timed(run[3100], 10) for _ in range(3)) / 1e3, 4)
        res["decode_M1_eager_us"] = round(timed(run[1], 200), 1)
        integrate.fuse_mlps(layer)
        integrate.fuse_linears(layer)
        integrate.fuse_rmsnorms(layer)
        integrate.fuse_add_rmsnorm(layer)
        integrate.fuse_text_rope()
        integrate.fuse_kv_rope(layer)
        saved_qo = integrate.TILED_MIN_ROWS_LINEAR
        try:
            # the fused prefill with this build's q/o choice and with the
            # reference's q/o rule (the tiled linear from 64 rows),
            # interleaved three times each after a warm-up (the first timed
            # group after injection read ~5% slow): medians
            for _ in range(10):
                run[3100]()
            pre = {saved_qo: [], 64: []}
            for r in range(6):
                rule = (saved_qo, 64)[r % 2]
                integrate.TILED_MIN_ROWS_LINEAR = rule
                pre[rule].append(timed(run[3100], 10))
            integrate.TILED_MIN_ROWS_LINEAR = saved_qo
            res["prefill_M3100_umic_ms"] = round(statistics.median(pre[saved_qo]) / 1e3, 4)
            res["prefill_M3100_umic_tiled_qo_ms"] = round(statistics.median(pre[64]) / 1e3, 4)
            res["decode_M1_umic_us"] = round(timed(run[1], 200), 1)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                run[1]()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                run[1]()
            res["decode_M1_umic_graph_us"] = round(timed(graph.replay, 200), 1)
        finally:
            integrate.TILED_MIN_ROWS_LINEAR = saved_qo
            integrate.unfuse_mlps(layer)
            integrate.unfuse_rope()
    return res


def vit_step(reps: int = 10) -> dict:
    """BASELINE config 4 in context: the Qwen3-VL vision encoder at the ViT
    width of the norm/RoPE rows (hidden 1280, 16 heads, head_dim 80, MLP
    1280 -> 5120 with the tanh GELU, 4 blocks, a deepstack tap after block 1)
    on 16 images of 32 x 32 patches -- 16384 tokens, the [16384, 1280]
    LayerNorm and [16384, 16, 80] vision-RoPE rows -- with random weights
    (LayerNorm affine 1 + N(0, 0.1) / N(0, 0.1)).  Timed eager, then with
    fuse_layernorms, fuse_vision_rope, fuse_vision_encoder_pipeline and
    fuse_gelu_mlps injected (the reference's vision set,
    src/umic/optimize.py:120-140, plus the fc1 + GELU epilogue)."""
    import torch
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLVisionConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLVisionModel

    from umic import integrate

    cfg = Qwen3VLVisionConfig(depth=4, hidden_size=1280, num_heads=16, intermediate_size=5120,
                              hidden_act="gelu_pytorch_tanh", patch_size=16,
                              temporal_patch_size=2, in_channels=3, spatial_merge_size=2,
                              out_hidden_size=2048, num_position_embeddings=2304,
                              deepstack_visual_indexes=[1], attn_implementation="sdpa")
    torch.manual_seed(0)
    m = Qwen3VLVisionModel(cfg)
    inv_freq = m.rotary_pos_emb.inv_freq.clone()
    m = m.to(torch.bfloat16)
    # a bf16 checkpoint keeps this fp32 buffer (HF builds it in fp32), so
    # cos/sin reach the RoPE in fp32, as in the model
    m.rotary_pos_emb.inv_freq = inv_freq
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, torch.nn.LayerNorm):
                mod.weight.add_(0.1 * torch.randn_like(mod.weight))
                mod.bias.add_(0.1 * torch.randn_like(mod.bias))
    m = m.to("cuda").eval()
    grid = torch.tensor([[1, 32, 32]] * 16, device="cuda")
    px = torch.randn(16 * 32 * 32, 3 * 2 * 16 * 16, device="cuda").to(torch.bfloat16)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps  # ms

    res = {"tokens": 16384, "blocks": 4}
    with torch.no_grad():
        run = lambda: m(px, grid_thw=grid)  # noqa: E731
        ref = run().last_hidden_state
        res["encoder_eager_ms"] = round(timed(run), 3)
        integrate.fuse_layernorms(m)
        integrate.fuse_vision_rope()
        integrate.fuse_vision_encoder_pipeline(m)
        integrate.fuse_gelu_mlps(m)
        try:
            out = run().last_hidden_state
            res["encoder_umic_ms"] = round(timed(run), 3)
            res["max_rel_err"] = round(float((out.float() - ref.float()).abs().max()
                                             / ref.float().abs().max()), 5)
        finally:
            integrate.unfuse_rope()
    return res


def kv_cache_step(reps: int = 20) -> dict:
    """Text RoPE fused with the in-place KV-cache append
    (umic_rope_kv_append_bf16) against the chain it replaces -- this
    library's q+k RoPE, then the cache's two slice assignments
    (src/umic/cache.py:69-70) -- at BASELINE config 5 head counts (32 q /
    8 kv heads, head_dim 128): a 3100-token prefill into an empty cache and a
    32-token flow step appended after a 3094-token prefix.  Inputs and caches
    rotate over rings of >= 640 MB so no launch is served from the Infinity
    Cache.  Algorithmic bytes: q, k, v read and written once, cos/sin read
    once: 2*2*(Hq+2*Hk)*S*D + 2*2*S*D."""
    import torch

    from umic.kernels import rope

    gen = torch.Generator(device="cuda").manual_seed(1)
    Hq, Hk, D, L = 32, 8, 128, 3200
    sa, sb = _bf(8192, 8192, gen=gen), _bf(8192, 8192, gen=gen)  # spacer GEMM operands
    res = {}
    for tag, S, pos in (("prefill_S3100", 3100, 0), ("flow_S32", 32, 3094)):
        inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        ang = torch.arange(pos, pos + S, dtype=torch.float32)[:, None] * inv[None]
        emb = torch.cat((ang, ang), -1)
        cos, sin = (f(emb).to(torch.bfloat16)[None].cuda() for f in (torch.cos, torch.sin))
        per_set = 2 * (Hq + 2 * Hk) * S * D + 2 * 2 * Hk * L * D
        n = max(2, min(32, int(-(-640e6 // per_set))))
        sets = [tuple(_bf(1, S, H, D, gen=gen).transpose(1, 2) for H in (Hq, Hk, Hk))
                + (torch.empty(1, Hk, L, D, dtype=torch.bfloat16, device="cuda"),
                   torch.empty(1, Hk, L, D, dtype=torch.bfloat16, device="cuda"))
                for _ in range(n)]

        def fused(i):
            q, k, v, kc, vc = sets[i % n]
            return rope.rope_kv_append(q, k, v, cos, sin, kc, vc, pos)

        def unfused(i):
            q, k, v, kc, vc = sets[i % n]
            qo, ko = rope.apply_rotary_text_hip(q, k, cos, sin)
            kc[:, :, pos:pos + S] = ko
            vc[:, :, pos:pos + S] = v
            return qo

        def timed(fn):
            """(GPU us per call, host us per call).  GPU time: the calls are
            queued behind ~2 ms of spacer GEMMs, so the events see device
            time only; host time: wall clock of back-to-back calls."""
            for i in range(3):
                fn(i)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            keep = [None] * n
            for _ in range(2):
                torch.matmul(sa, sb)
            e0.record()
            for i in range(reps):
                keep[i % n] = fn(i)
            e1.record()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(reps):
                keep[i % n] = fn(i)
            host = (time.perf_counter() - t0) / reps * 1e6
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / reps * 1e3, host

        nbytes = 2 * 2 * (Hq + 2 * Hk) * S * D + 2 * 2 * S * D
        (us_f, host_f), (us_u, host_u) = timed(fused), timed(unfused)
        res[tag] = {"fused_us": round(us_f, 2), "unfused_us": round(us_u, 2),
                    "fused_host_us": round(host_f, 1), "unfused_host_us": round(host_u, 1),
                    "bytes": nbytes, "gbps": round(nbytes / (us_f * 1e-6) / 1e9, 1),
                    "frac": round(nbytes / (us_f * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                    "ring": n}
        del sets
    return res


def vit_sites() -> int:
    """The ViT projection sites the reference left on the vendor library
    (src/umic/integrate.py:93-95, 261-319), this library's linear against
    hipBLASLt at M=16384 tokens, hidden 1280: one JSON line per site."""
    import torch

    from umic import _lib
    from umic.kernels import linear

    _lib.load()
    torch.cuda.set_device(0)
    F = torch.nn.functional

    def timed(fn, reps=30):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3

    M = 16384
    approx = {"gelu": "none", "gelu_tanh": "tanh"}
    for site, K, N, act in (("qkv", 1280, 3840, None), ("fc1_gelu", 1280, 5120, "gelu"),
                            ("fc1_gelu_tanh", 1280, 5120, "gelu_tanh"),
                            ("fc2", 5120, 1280, None)):
        x = _bf(M, K)
        w, b = _bf(N, K, scale=0.02), _bf(N, scale=0.1)
        ours = timed(lambda: linear.linear_hip(x, w, b, act=act))
        if act:
            vendor = timed(lambda: F.gelu(F.linear(x, w, b), approximate=approx[act]))
        else:
            vendor = timed(lambda: F.linear(x, w, b))
        print(json.dumps({"site": site, "M": M, "K": K, "N": N, "act": act,
                          "umic_us": round(ours, 1), "vendor_us": round(vendor, 1),
                          "umic_tflops": round(2 * M * N * K / ours / 1e6, 1)}), flush=True)
    # the whole ViT MLP block as fuse_gelu_mlps runs it (fc1 + bias + GELU in
    # one launch, fc2 on the vendor library) against the eager block
    H, I = 1280, 5120
    x = _bf(M, H)
    w1, b1 = _bf(I, H, scale=0.02), _bf(I, scale=0.1)
    w2, b2 = _bf(H, I, scale=0.02), _bf(H, scale=0.1)
    for act in ("gelu_tanh", "gelu"):
        ours = timed(lambda: F.linear(linear.linear_hip(x, w1, b1, act=act), w2, b2))
        eager = timed(lambda: F.linear(F.gelu(F.linear(x, w1, b1), approximate=approx[act]),
                                       w2, b2))
        print(json.dumps({"site": f"mlp_block_{act}", "M": M, "hidden": H, "intermediate": I,
                          "umic_us": round(ours, 1), "eager_us": round(eager, 1),
                          "speedup": round(eager / ours, 3)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-sample-s", type=float, default=6.0,
                    help="seconds of scalar-oracle timing (cpu_oracle)")
    ap.add_argument("--cpu-budget-s", type=float, default=45.0,
                    help="seconds the reference's eager CPU path may take (cpu_baseline)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-only", action="store_true",
                    help="print only the CPU baselines (no GPU needed)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="one launch per kernel after a calibration copy, for rocprofv3 --pmc")
    ap.add_argument("--probe-only", default=None,
                    help="with --pmc-probe: comma-separated bench entries to launch "
                         "(after the calibration copy)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="take roofline.traffic from the committed PMC summary instead of "
                         "measuring it (three rocprofv3 --pmc child runs); use when this run "
                         "is itself under rocprofv3")
    ap.add_argument("--copy-ceiling", action="store_true",
                    help="time plain device copies of the norm/RoPE byte counts")
    ap.add_argument("--vit-sites", action="store_true",
                    help="time the ViT projection sites, this library against hipBLASLt")
    ap.add_argument("--decode-layer", action="store_true",
                    help="run ten fused config-5 decode steps (for a kernel trace) and exit")
    ap.add_argument("--decode-gemv", action="store_true",
                    help="time the config-5 decode GEMVs on cold weights against plain reads "
                         "of the same bytes, print them and exit")
    ap.add_argument("--no-layer", action="store_true",
                    help="skip the decoder-layer (config 5) and vision-encoder (config 4) "
                         "timings")
    ap.add_argument("--no-kv-cache", action="store_true",
                    help="skip the fused RoPE + KV-cache append timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the norm "
              "and RoPE kernels would shard along M (tokens) with no exchange, and the "
              "GEMMs by weight columns with one all-reduce after down_proj and o_proj",
              file=sys.stderr)
        return 2

    if args.cpu_only:
        print(json.dumps({"cpu_baseline": cpu_reference(args.cpu_budget_s),
                          "cpu_oracle": cpu_oracle(args.cpu_sample_s)}), flush=True)
        return 0
    if args.pmc_probe:
        return pmc_probe(args.probe_only.split(",") if args.probe_only else None)
    if args.copy_ceiling:
        return copy_ceiling()
    if args.vit_sites:
        return vit_sites()
    if args.decode_layer:
        return decode_layer()
    if args.decode_gemv:
        import torch

        from umic import _lib

        _lib.load()
        torch.cuda.set_device(0)
        print(json.dumps({"decode_gemv": decode_gemv_step()}), flush=True)
        return 0

    import torch

    from umic import _lib

    _lib.load()
    torch.cuda.set_device(0)
    ents, rings, spacer = build_workload()
    torch.cuda.synchronize()

    for i in range(args.warmup):
        for _, fn, *_ in ents:
            fn(i)
    torch.cuda.synchronize()

    K = args.steps
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in ents]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for j, (name, fn, *_) in enumerate(ents):
        n = rings.get(name, 1)
        keep = [None] * n  # outputs live for one ring turn
        # an untimed ring turn first: the outputs' blocks exist before the
        # first event, and the timed launches reuse them as each output is
        # replaced (without it the first timed group paid for new device
        # allocations: rmsnorm read 20-74 us instead of 10.5 in such runs)
        for s in range(n):
            keep[s] = fn(s)
        spacer()
        spacer()
        evs[j][0].record()
        for s in range(n, n + K):
            keep[s % n] = fn(s)
        evs[j][1].record()
        del keep
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    kern = {}
    for j, (name, _, nbytes, flops, bound) in enumerate(ents):
        us = evs[j][0].elapsed_time(evs[j][1]) / K * 1e3
        rec = {"us": round(us, 2), "bound": bound, "bytes": nbytes}
        rec["gbps"] = round(nbytes / (us * 1e-6) / 1e9, 1)
        if bound == "hbm":
            rec["frac"] = round(rec["gbps"] / HBM_PEAK_GBS, 4)
        else:
            rec["flops"] = flops
            rec["tflops"] = round(flops / (us * 1e-6) / 1e12, 1)
            rec["frac"] = round(rec["tflops"] / BF16_PEAK_TFLOPS, 4)
        kern[name] = rec

    # each HBM-bound kernel against a plain device copy of its byte count,
    # timed the same way right after the kernels: of_copy = copy time / kernel
    # time (1.0 = as fast as the runtime's own copy of those bytes)
    copy_us = {}
    for name, rec in kern.items():
        if rec["bound"] == "hbm":
            if rec["bytes"] not in copy_us:
                copy_us[rec["bytes"]] = same_bytes_copy(rec["bytes"], K, spacer)
            c = copy_us[rec["bytes"]]
            rec["copy_us"] = round(c, 2)
            rec["copy_gbps"] = round(rec["bytes"] / (c * 1e-6) / 1e9, 1)
            rec["of_copy"] = round(c / rec["us"], 3)
    # and against the library's tuned streaming copy of the same bytes
    tuned_us = {}
    for name, rec in kern.items():
        if rec["bound"] == "hbm":
            if rec["bytes"] not in tuned_us:
                tuned_us[rec["bytes"]] = stream_copy_us(rec["bytes"], K, spacer)
            c = tuned_us[rec["bytes"]]
            rec["stream_copy_us"] = round(c, 2)
            rec["stream_copy_gbps"] = round(rec["bytes"] / (c * 1e-6) / 1e9, 1)
            rec["of_stream_copy"] = round(c / rec["us"], 3)

    hbm = [kern[n] for n in VALUE_SITES]
    agg = sum(k["bytes"] for k in hbm) / (sum(k["us"] for k in hbm) * 1e-6) / 1e9
    mlp_ms = (kern["gate_silu_mul"]["us"] + kern["down_proj"]["us"]) / 1e3
    dom_name = max((n for n in kern if not n.endswith("_vendor")), key=lambda n: kern[n]["us"])
    dom = kern[dom_name]
    if dom["bound"] == "hbm":
        roof = {"kernel": dom_name, "bound": "hbm", "achieved": dom["gbps"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": dom["frac"]}
    else:
        roof = {"kernel": dom_name, "bound": "mfma", "achieved": dom["tflops"],
                "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": dom["frac"]}
    # every other measurement first: after the profiler's child runs, some of
    # this process's later kernels ran slower (the fused ViT encoder 25 against
    # 10 ms), so the PMC passes come last
    layer = None if args.no_layer else layer_step()
    decode = None if args.no_layer else decode_gemv_step()
    vit = None if args.no_layer else vit_step()
    kv = None if args.no_kv_cache else kv_cache_step()
    cpu_base = None if args.no_cpu_baseline else cpu_reference(args.cpu_budget_s)
    cpu_port = None if args.no_cpu_baseline else cpu_oracle(args.cpu_sample_s)
    traffic, scales, why = (None, None, "--no-traffic") if args.no_traffic else \
        measure_traffic(dom_name)
    if traffic is not None:
        roof["traffic"] = traffic
        roof["traffic_source"] = ("measured in this run: rocprofv3 --pmc FETCH_SIZE, then "
                                  "WRITE_SIZE, over bench.py --pmc-probe --probe-only "
                                  f"{dom_name}; counters scaled by a {COPY_BYTES >> 20} MiB "
                                  "device copy")
        roof["traffic_counters"] = scales
        # the clock: GUI-active cycles per XCD (32 CUs each) over the
        # kernel's timed duration
        import torch

        xcds = max(1, torch.cuda.get_device_properties(0).multi_processor_count // 32)
        roof["clock_ghz"] = round(scales["grbm_gui_active"] / xcds / (dom["us"] * 1e3), 3)
        roof["clock_source"] = (f"GRBM_GUI_ACTIVE {scales['grbm_gui_active']:.0f} over {xcds} "
                                f"XCDs / {dom['us']} us (rocprofv3 --pmc GRBM_GUI_ACTIVE pass "
                                "of the same probe)")
    else:
        roof["traffic"] = load_traffic(dom_name)
        roof["traffic_source"] = (f"committed profiles/traffic_{dom_name}.json (not measured "
                                  f"in this run: {why})")
    roof["algorithmic_bytes"] = dom["bytes"]

    out = {
        "metric": METRIC,
        "value": round(agg, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(sum(v["us"] for n, v in kern.items() if not n.endswith("_vendor"))
                             / 1e3, 3),
        "wall_ms_per_step": round(wall / K * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "BASELINE configs 2-4 at full size: norms [3100,4096] and "
                               "[16384,1280], RoPE text q/k [1,32|8,3100,128] and vision "
                               "[16384,16,80], q/o proj and P5 MLP at M=3100 K=4096 N=4096|12288, "
                               "down_proj K=12288 N=4096",
                   "rows_lm": 3100, "rows_vit": 16384, "input_rings": rings},
        "hbm_frac": round(agg / HBM_PEAK_GBS, 4),
        # the same six kernels against same-size device copies (kernels[..]
        # .copy_us): aggregate copy GB/s over those byte counts, and the
        # kernels' aggregate as a fraction of it
        "copy_ceiling_gbps": round(sum(k["bytes"] for k in hbm)
                                   / (sum(k["copy_us"] for k in hbm) * 1e-6) / 1e9, 1),
        "of_copy": round(sum(k["copy_us"] for k in hbm) / sum(k["us"] for k in hbm), 3),
        # and against the library's tuned streaming copy (.stream_copy_us)
        "stream_copy_ceiling_gbps": round(sum(k["bytes"] for k in hbm)
                                          / (sum(k["stream_copy_us"] for k in hbm) * 1e-6)
                                          / 1e9, 1),
        "of_stream_copy": round(sum(k["stream_copy_us"] for k in hbm)
                                / sum(k["us"] for k in hbm), 3),
        "mlp_prefill_ms": round(mlp_ms, 4),
        "kernels": kern,
        "roofline": roof,
        "layer": layer,
        "decode_gemv": decode,
        "vit_encoder": vit,
        "kv_cache": kv,
        "cpu_baseline": cpu_base,
        "cpu_oracle": cpu_port,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
