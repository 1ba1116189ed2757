"""GPU: umic_linear_sk_static_bf16, the stream-K linear on the library's
static scratch (no workspace argument, no allocation).

Through the C ABI, against umic_linear_ws_bf16 on a caller workspace (the
same kernel, so bit for bit): stream-K calls in a row on one stream, each
smaller than the one before (the BASELINE down_proj on the four-wave
schedule, 63.8 MiB; then 96 tiles of the eight-wave one; the last with a
bias and the GELU epilogue), so each runs on the scratch the previous left
behind; a few-row (GEMV) and a data-parallel
shape, which need no scratch and pass through to umic_linear_bf16; and a
shape whose workspace exceeds the 64 MiB scratch, rejected before any
launch.
"""

from __future__ import annotations

import pytest
import torch
from helpers import bf16_randn, max_rel_err

from umic import _lib
from umic.kernels import linear

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCRATCH_BYTES = 64 << 20


def _operands(M, N, K, seed, bias=False):
    g = torch.Generator().manual_seed(seed)
    x = bf16_randn(M, K, gen=g).to(DEV)
    w = bf16_randn(N, K, scale=0.02, gen=g).to(DEV)
    b = bf16_randn(N, scale=0.1, gen=g).to(DEV) if bias else None
    return x, w, b


def _static(x, w, b, act):
    M, K = x.shape
    N = w.shape[0]
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    _lib.call("umic_linear_sk_static_bf16", x.data_ptr(), w.data_ptr(), _lib.ptr(b),
              out.data_ptr(), M, N, K, K, K, N, act, _lib.stream_of(x))
    return out


def _with_workspace(x, w, b, act):
    M, K = x.shape
    N = w.shape[0]
    need = _lib.lib().umic_linear_workspace_bytes(M, N, K)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=DEV)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    _lib.call("umic_linear_ws_bf16", x.data_ptr(), w.data_ptr(), _lib.ptr(b), out.data_ptr(),
              M, N, K, K, K, N, act, ws.data_ptr(), ws.numel(), _lib.stream_of(x))
    return out


def test_static_scratch_matches_the_workspace_entry_point():
    calls = [((3100, 4096, 12288), 7, False, _lib.UMIC_ACT_NONE),
             ((1536, 4096, 12288), 1, False, _lib.UMIC_ACT_NONE),
             ((300, 4096, 12288), 6, False, _lib.UMIC_ACT_NONE),
             ((32, 2048, 12288), 2, True, _lib.UMIC_ACT_GELU)]
    for (M, N, K), seed, bias, act in calls:
        need = _lib.lib().umic_linear_workspace_bytes(M, N, K)
        print(f"static stream-K M={M} N={N} K={K} act={act} bias={bias} ws={need}", flush=True)
        assert 0 < need <= SCRATCH_BYTES
        x, w, b = _operands(M, N, K, seed, bias)
        assert linear.stream_k_planned(x, w)
        got = _static(x, w, b, act)
        ref = _with_workspace(x, w, b, act)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, N, K)
        eager = x.float() @ w.float().t() + (b.float() if bias else 0)
        if act == _lib.UMIC_ACT_GELU:
            eager = torch.nn.functional.gelu(eager)
        assert max_rel_err(got, eager) <= 2e-2


@pytest.mark.parametrize("M,N,K", [(4, 1024, 4096), (600, 1024, 8192)])
def test_shapes_without_scratch_pass_through(M, N, K):
    """The GEMV and the data-parallel kernel need no scratch: the static
    entry point gives umic_linear_bf16's result."""
    print(f"pass-through M={M} N={N} K={K}", flush=True)
    assert _lib.lib().umic_linear_workspace_bytes(M, N, K) == 0
    x, w, _ = _operands(M, N, K, 3)
    got = _static(x, w, None, _lib.UMIC_ACT_NONE)
    ref = torch.empty_like(got)
    _lib.call("umic_linear_bf16", x.data_ptr(), w.data_ptr(), None, ref.data_ptr(), M, N, K,
              K, K, N, _lib.UMIC_ACT_NONE, _lib.stream_of(x))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_shape_beyond_the_scratch_is_rejected():
    M, N, K = 2048, 4096, 12288  # 128 output tiles: 64 MiB of partials plus the counters
    assert _lib.lib().umic_linear_workspace_bytes(M, N, K) > SCRATCH_BYTES
    x, w, _ = _operands(M, N, K, 4)
    out = torch.zeros(M, N, dtype=torch.bfloat16, device=DEV)
    rc = _lib.lib().umic_linear_sk_static_bf16(x.data_ptr(), w.data_ptr(), None, out.data_ptr(),
                                               M, N, K, K, K, N, _lib.UMIC_ACT_NONE,
                                               _lib.stream_of(x))
    assert rc == _lib.UMIC_ERR_SCRATCH
    assert "64 MiB" in _lib.error_string(rc)
    torch.cuda.synchronize()
    assert not out.any()  # nothing ran


@pytest.mark.parametrize("M", [300, 3100])
def test_static_scratch_under_graph_capture(M):
    """The static entry point captured in a HIP graph (its callers are code
    under capture): every replay, with new inputs copied in and eager work
    between replays, equals the workspace entry point bit for bit -- on the
    eight-wave stream-K schedule (M = 300) and the four-wave one (the
    BASELINE down_proj, M = 3100)."""
    N, K = 4096, 12288
    print(f"static stream-K graph capture M={M} N={N} K={K}", flush=True)
    x, w, _ = _operands(M, N, K, 5)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)

    def launch():
        _lib.call("umic_linear_sk_static_bf16", x.data_ptr(), w.data_ptr(), None,
                  out.data_ptr(), M, N, K, K, K, N, _lib.UMIC_ACT_NONE, _lib.stream_of(x))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()                      # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    for seed in (6, 7, 8):
        x2, _, _ = _operands(M, N, K, seed)
        x.copy_(x2)
        graph.replay()
        torch.cuda.synchronize()
        ref = _with_workspace(x, w, None, _lib.UMIC_ACT_NONE)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), seed
