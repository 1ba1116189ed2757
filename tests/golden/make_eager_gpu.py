"""Record torch-ROCm eager's fp32 row statistics on the GPU (run on the box).

The eager norms the kernels replace compute their row statistics on the GPU
in fp32, in an order fixed by torch's reduction kernels:

  RMSNorm    HF Qwen3VLTextRMSNorm: v = x.float().pow(2).mean(-1); rstd =
             torch.rsqrt(v + eps)  (transformers modeling_qwen3_vl.py:400-405)
  LayerNorm  torch.nn.functional.layer_norm -> aten native_layer_norm, whose
             second and third outputs are the fp32 row mean and rstd

A bf16 output of either op can move by one ulp when a statistic moves by one
fp32 ulp, so parity within one bf16 ulp of eager needs these statistics
bit-exact.  This script evaluates them with torch on the GPU for seeded
inputs (drawn on the CPU exactly as tests/helpers.py:bf16_randn does, so the
inputs are regenerated bit for bit from the seed anywhere) and stores them,
with eager's bf16 outputs for a few rows and a sweep of torch.rsqrt, as
numpy arrays (statistics of the leading 1024 rows, outputs of the leading 4).
tests/test_oracle.py checks the oracle against the committed copy
(tests/golden/eager_gpu_stats.npz).

    python tests/golden/make_eager_gpu.py OUT.npz
"""

from __future__ import annotations

import sys

import numpy as np
import torch

# (rows, n, seed) of the RMSNorm statistic cases: the BASELINE shapes (LM
# rows [3100, 4096], q_norm / k_norm head rows [99200, 128] / [24800, 128]),
# decode rows, and every row-count regime of torch's reduction launch
# (1, 2-3, 4-7, >= 8 rows per block) at several widths.
RMS_CASES = [(3100, 4096, 0), (99200, 128, 1), (24800, 128, 2), (1, 4096, 3), (2, 4096, 4),
             (3, 4096, 5), (4, 4096, 6), (5, 4096, 7), (7, 4096, 8), (8, 4096, 9),
             (9, 4096, 10), (64, 4096, 11), (257, 4096, 12), (32, 128, 13), (8, 128, 14),
             (1, 128, 15), (333, 1280, 16), (16, 2048, 17), (16, 2560, 18), (16, 5120, 19),
             (4, 8192, 20), (16, 8192, 21), (64, 1000, 22), (77, 80, 23), (31, 100, 24),
             (1, 1280, 25), (3, 1152, 26)]
# (rows, n, seed) of the LayerNorm cases: the ViT rows [16384, 1280] and
# others around the kernel's launch regimes.
LN_CASES = [(16384, 1280, 100), (4096, 1152, 101), (1, 1280, 102), (7, 1280, 103),
            (64, 1280, 104), (100, 4096, 105), (64, 1000, 106), (16390, 128, 107),
            (50, 80, 108), (13, 100, 109), (8, 8192, 110), (3, 4096, 111), (256, 2048, 112)]
# (rows, n, seed, offset) of the LayerNorm cases eager runs with its scalar
# kernel (RowwiseMomentsCUDAKernel, then LayerNormForwardCUDAKernel): widths
# that are not a multiple of 4, and (offset 1) a contiguous input starting one
# element past an aligned buffer, which defeats the vectorized kernel's
# alignment check.
LN_SCALAR_CASES = [(4999, 127, 200, 0), (64, 1001, 201, 0), (7, 6, 202, 0), (13, 130, 203, 0),
                   (100, 2050, 204, 0), (3, 4097, 205, 0), (257, 1282, 206, 0), (5, 1, 207, 0),
                   (64, 1280, 208, 1), (9, 4096, 209, 1), (33, 100, 210, 1)]
KEEP_ROWS = 4  # eager bf16 outputs kept per case (leading rows)
STAT_ROWS = 1024  # row statistics kept per case (leading rows)


def draw(rows: int, n: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, n, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
    b = (0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
    return x, w, b


def u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16).copy()


def main(out: str) -> None:
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextRMSNorm

    dev = "cuda"
    res: dict[str, np.ndarray] = {}
    eps = 1e-6
    with torch.no_grad():
        for rows, n, seed in RMS_CASES:
            x, w, _ = draw(rows, n, seed)
            xd = x.to(dev)
            var = xd.to(torch.float32).pow(2).mean(-1, keepdim=True)
            rstd = torch.rsqrt(var + eps)
            m = Qwen3VLTextRMSNorm(n, eps=eps).to(device=dev, dtype=torch.bfloat16)
            m.weight.copy_(w.to(dev))
            y = m(xd)
            key = f"rms_{rows}x{n}"
            res[key + "_var"] = var.view(-1)[:STAT_ROWS].cpu().numpy()
            res[key + "_rstd"] = rstd.view(-1)[:STAT_ROWS].cpu().numpy()
            res[key + "_y"] = u16(y[:KEEP_ROWS])
            res[key + "_xsum"] = np.array([int(u16(x).astype(np.uint64).sum())], np.uint64)
            print(key, flush=True)
        # the HF module on its real [B, S, H, D] head-row view and [B, S, hidden] rows
        x, w, _ = draw(3100 * 32, 128, 1)
        xd = x.to(dev).view(1, 3100, 32, 128)
        res["rms_q4d_var"] = xd.to(torch.float32).pow(2).mean(-1).view(-1)[:STAT_ROWS].cpu().numpy()
        x, w, _ = draw(3100, 4096, 0)
        xd = x.to(dev).view(1, 3100, 4096)
        res["rms_h3d_var"] = xd.to(torch.float32).pow(2).mean(-1).view(-1)[:STAT_ROWS].cpu().numpy()

        for rows, n, seed in LN_CASES:
            x, w, b = draw(rows, n, seed)
            y, mean, rstd = torch.ops.aten.native_layer_norm(x.to(dev), [n], w.to(dev),
                                                              b.to(dev), eps)
            key = f"ln_{rows}x{n}"
            res[key + "_mean"] = mean.view(-1)[:STAT_ROWS].float().cpu().numpy()
            res[key + "_rstd"] = rstd.view(-1)[:STAT_ROWS].float().cpu().numpy()
            res[key + "_y"] = u16(y[:KEEP_ROWS])
            res[key + "_stat_dtype"] = np.array([str(mean.dtype)])
            print(key, flush=True)

        for rows, n, seed, off in LN_SCALAR_CASES:
            x, w, b = draw(rows, n, seed)
            flat = torch.empty(rows * n + off, dtype=torch.bfloat16, device=dev)
            flat[off:] = x.to(dev).view(-1)
            xd = flat[off:].view(rows, n)
            y, mean, rstd = torch.ops.aten.native_layer_norm(xd, [n], w.to(dev), b.to(dev), eps)
            key = f"lns_{rows}x{n}_o{off}"
            res[key + "_mean"] = mean.view(-1)[:STAT_ROWS].float().cpu().numpy()
            res[key + "_rstd"] = rstd.view(-1)[:STAT_ROWS].float().cpu().numpy()
            res[key + "_y"] = u16(y[:KEEP_ROWS])
            print(key, flush=True)

        # torch.rsqrt over every fp32 mantissa of [1, 4) and a log-uniform
        # sample, against the correctly rounded value (fp64 rsqrt, rounded)
        ar = torch.arange(1 << 23, dtype=torch.int64)
        sets = {"m1": (ar + (127 << 23)).to(torch.int32).view(torch.float32),
                "m2": (ar + (128 << 23)).to(torch.int32).view(torch.float32)}
        g = torch.Generator().manual_seed(7)
        sets["log"] = torch.exp(torch.empty(1 << 22).uniform_(-30.0, 30.0, generator=g))
        for name, xs in sets.items():
            xd = xs.to(dev)
            got = torch.rsqrt(xd)
            cr = (1.0 / torch.sqrt(xd.double())).float()
            bad = (got.view(torch.int32) != cr.view(torch.int32)).nonzero().view(-1)
            res[f"rsqrt_{name}_n"] = np.array([xs.numel()], np.int64)
            res[f"rsqrt_{name}_bad_x"] = xs[bad.cpu()][:1000].numpy()
            res[f"rsqrt_{name}_bad_got"] = got[bad][:1000].cpu().numpy()
            inv = (1.0 / torch.sqrt(xd))  # fp32 sqrt then fp32 division
            res[f"rsqrt_{name}_vs_divsqrt"] = np.array(
                [int((inv.view(torch.int32) != got.view(torch.int32)).sum())], np.int64)
            print(f"rsqrt {name}: {bad.numel()} of {xs.numel()} differ from CR", flush=True)
        res["torch_version"] = np.array([torch.__version__])
        res["hip_version"] = np.array([str(torch.version.hip)])
        res["device"] = np.array([torch.cuda.get_device_name(0)])
    np.savez_compressed(out, **res)
    print("wrote", out, flush=True)


if __name__ == "__main__":
    main(sys.argv[1])
