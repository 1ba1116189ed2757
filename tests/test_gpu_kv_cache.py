"""GPU parity: text RoPE fused with the in-place KV-cache append
(``umic_rope_kv_append_bf16`` through ``umic.kernels.rope.rope_kv_append`` and
``umic.cache.InplaceLayer.append_rotary``).

q/k/v are laid out as transformers' qwen3_vl text attention hands them over
(transposed [B,H,S,D] views of [B,S,H,D] projections), caches are
[B, Hkv, capacity, D] buffers pre-filled with random sentinel values.
Checked bit for bit: rope(q) and the k rows written into the cache against
the CPU oracle, the v rows against v, and every other cache row against its
sentinel.  Shapes: a 3100-token prefill into a fresh cache, a 32-token flow
step after the 3094-token prefix, a decode token, a batch of two with
per-sequence tables, and an append that exactly fills the cache.
"""

from __future__ import annotations

import collections

import numpy as np
import pytest
import torch
from helpers import bf16_randn, bits, max_rel_err, qwen3_decoder_layer, rel_err, ulp

import oracle
from umic import _lib, integrate
from umic.cache import InplaceKVCache
from umic.kernels import rope

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::FutureWarning")]
DEV = "cuda"


def tables(B, S, D, pos):
    """bf16 text cos/sin [B, S, D] for positions pos.. (+3 per batch row)."""
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextRotaryEmbedding

    cfg = Qwen3VLTextConfig(hidden_size=8 * D, num_attention_heads=8, num_key_value_heads=8,
                            head_dim=D, rope_parameters={"rope_type": "default",
                                                         "rope_theta": 1e6})
    ids = torch.stack([torch.arange(pos + 3 * b, pos + 3 * b + S) for b in range(B)])
    return Qwen3VLTextRotaryEmbedding(cfg)(torch.zeros(1, dtype=torch.bfloat16), ids)


def inputs(B, S, Hq, Hk, D, L, seed):
    g = torch.Generator().manual_seed(seed)
    qs, ks, vs = (bf16_randn(B, S, H, D, gen=g) for H in (Hq, Hk, Hk))   # [B, S, H, D]
    kc0, vc0 = bf16_randn(B, Hk, L, D, gen=g), bf16_randn(B, Hk, L, D, gen=g)
    return qs, ks, vs, kc0, vc0


def check(qo, kc, vc, qs, ks, vs, kc0, vc0, cos, sin, rows):
    """rows[b] = cache positions written for sequence position 0..S-1."""
    qo, kc, vc = bits(qo.transpose(1, 2)), bits(kc), bits(vc)
    for b in range(qs.shape[0]):
        c, s = bits(cos)[b], bits(sin)[b]
        assert np.array_equal(qo[b], oracle.rope_text(bits(qs)[b], c, s))
        krot = oracle.rope_text(bits(ks)[b], c, s)            # [S, Hk, D]
        for i, t in enumerate(rows):
            if t is None:
                continue
            assert np.array_equal(kc[b][:, t], krot[i]), (b, i, t)
            assert np.array_equal(vc[b][:, t], bits(vs)[b][i]), (b, i, t)
    untouched = np.ones(kc.shape[2], bool)
    untouched[[t for t in rows if t is not None]] = False
    assert np.array_equal(kc[:, :, untouched], bits(kc0)[:, :, untouched])
    assert np.array_equal(vc[:, :, untouched], bits(vc0)[:, :, untouched])


@pytest.mark.parametrize("B,S,Hq,Hk,D,pos,L", [
    (1, 3100, 32, 8, 128, 0, 3200),      # prefill into a fresh cache
    (1, 32, 32, 8, 128, 3094, 3200),     # flow step after the 3094-token prefix
    (1, 1, 32, 8, 128, 3126, 3200),      # decode token
    (2, 5, 4, 2, 64, 7, 16),             # batch of two, per-sequence tables
    (1, 9, 3, 1, 16, 0, 9),              # exactly fills the cache
])
def test_rope_kv_append_vs_oracle(B, S, Hq, Hk, D, pos, L):
    print(f"rope_kv_append B={B} S={S} Hq={Hq} Hk={Hk} D={D} pos={pos} L={L}", flush=True)
    qs, ks, vs, kc0, vc0 = inputs(B, S, Hq, Hk, D, L, seed=S + D)
    cos, sin = tables(B, S, D, pos)
    q, k, v = (t.to(DEV).transpose(1, 2) for t in (qs, ks, vs))
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    qo = rope.rope_kv_append(q, k, v, cos.to(DEV), sin.to(DEV), kc, vc, pos)
    torch.cuda.synchronize()
    assert qo.shape == q.shape and qo.stride() == q.stride()
    check(qo, kc, vc, qs, ks, vs, kc0, vc0, cos, sin, list(range(pos, pos + S)))
    # the same as transformers' RoPE followed by the cache's slice assignment
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb

    rq, rk = apply_rotary_pos_emb(q, k, cos.to(DEV), sin.to(DEV))
    assert torch.equal(qo, rq) and torch.equal(kc[:, :, pos:pos + S], rk)


def test_known_position_past_the_cache_raises():
    qs, ks, vs, kc0, vc0 = inputs(1, 4, 2, 1, 32, 8, seed=3)
    cos, sin = tables(1, 4, 32, 0)
    q, k, v = (t.to(DEV).transpose(1, 2) for t in (qs, ks, vs))
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    with pytest.raises(RuntimeError, match="overflow"):
        rope.rope_kv_append(q, k, v, cos.to(DEV), sin.to(DEV), kc, vc, 5)
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), kc0) and torch.equal(vc.cpu(), vc0)


def test_device_position_rows_outside_the_cache_are_dropped():
    B, S, Hq, Hk, D, L = 1, 4, 2, 1, 32, 8
    qs, ks, vs, kc0, vc0 = inputs(B, S, Hq, Hk, D, L, seed=4)
    cos, sin = tables(B, S, D, 0)
    q, k, v = (t.to(DEV).transpose(1, 2) for t in (qs, ks, vs))
    for p, rows in ((6, [6, 7, None, None]), (L, [None] * 4), (-2, [None, None, 0, 1])):
        kc, vc = kc0.to(DEV), vc0.to(DEV)
        pos_t = torch.tensor([p], dtype=torch.int64, device=DEV)
        qo = rope.rope_kv_append(q, k, v, cos.to(DEV), sin.to(DEV), kc, vc, 0, pos_t)
        torch.cuda.synchronize()
        check(qo, kc, vc, qs, ks, vs, kc0, vc0, cos, sin, rows)


def test_device_position_replays_in_a_captured_graph():
    """Decode-graph use: one capture, every replay appends one token at the
    position held in device memory (the replay-safe form of the reference's
    index_copy_, src/umic/cache.py:53-63)."""
    B, S, Hq, Hk, D, L = 1, 1, 32, 8, 128, 64
    _, _, _, kc0, vc0 = inputs(B, S, Hq, Hk, D, L, seed=5)
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    qs_buf = torch.zeros(B, S, Hq, D, dtype=torch.bfloat16, device=DEV)
    ks_buf = torch.zeros(B, S, Hk, D, dtype=torch.bfloat16, device=DEV)
    vs_buf = torch.zeros(B, S, Hk, D, dtype=torch.bfloat16, device=DEV)
    cos_buf = torch.zeros(B, S, D, dtype=torch.bfloat16, device=DEV)
    sin_buf = torch.zeros_like(cos_buf)
    pos_t = torch.zeros(1, dtype=torch.int64, device=DEV)
    q, k, v = qs_buf.transpose(1, 2), ks_buf.transpose(1, 2), vs_buf.transpose(1, 2)

    def step():
        return rope.rope_kv_append(q, k, v, cos_buf, sin_buf, kc, vc, 0, pos_t)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()                                  # warm-up write at row 0
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qo = step()
    torch.cuda.synchronize()
    kc0 = kc.cpu()                              # sentinel state after the warm-up
    vc0 = vc.cpu()
    written = {}
    for n, p in enumerate((5, 6, 7, 63)):
        qs, ks, vs, _, _ = inputs(B, S, Hq, Hk, D, L, seed=100 + n)
        cos, sin = tables(B, S, D, p)
        for buf, src in ((qs_buf, qs), (ks_buf, ks), (vs_buf, vs), (cos_buf, cos),
                         (sin_buf, sin)):
            buf.copy_(src.to(DEV))
        pos_t.fill_(p)
        graph.replay()
        torch.cuda.synchronize()
        krot = oracle.rope_text(bits(ks)[0], bits(cos)[0], bits(sin)[0])
        assert np.array_equal(bits(qo.transpose(1, 2))[0],
                              oracle.rope_text(bits(qs)[0], bits(cos)[0], bits(sin)[0]))
        written[p] = (krot[0], bits(vs)[0][0])
        for t, (kr, vr) in written.items():     # earlier replays' rows persist
            assert np.array_equal(bits(kc)[0][:, t], kr) and np.array_equal(bits(vc)[0][:, t], vr)
    rest = np.ones(L, bool)
    rest[list(written)] = False
    assert np.array_equal(bits(kc)[:, :, rest], bits(kc0)[:, :, rest])
    assert np.array_equal(bits(vc)[:, :, rest], bits(vc0)[:, :, rest])


def test_inplace_layer_replay_append_matches_update():
    """InplaceLayer.append_rotary during replay = transformers RoPE +
    InplaceLayer.update (index_copy_ at the device cursor)."""
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb

    from transformers.cache_utils import DynamicCache

    B, Hq, Hk, D, base = 1, 32, 8, 128, 40
    g = torch.Generator().manual_seed(6)
    prefix_k = bf16_randn(B, Hk, base, D, gen=g).to(DEV)
    prefix_v = bf16_randn(B, Hk, base, D, gen=g).to(DEV)
    caches = []
    for _ in range(2):
        dyn = DynamicCache()
        dyn.update(prefix_k, prefix_v, 0)
        c = InplaceKVCache.from_dynamic(dyn, extra_tokens=8)
        # the token goes right after the prefix, so rows [0, base] are all
        # defined and the replay window covers exactly them
        c.replay_at(torch.tensor([base], dtype=torch.int64, device=DEV), base + 1)
        caches.append(c)
    q = bf16_randn(B, 1, Hq, D, gen=g).to(DEV).transpose(1, 2)
    k = bf16_randn(B, 1, Hk, D, gen=g).to(DEV).transpose(1, 2)
    v = bf16_randn(B, 1, Hk, D, gen=g).to(DEV).transpose(1, 2)
    cos, sin = (t.to(DEV) for t in tables(B, 1, D, base))
    lyr_a, lyr_b = caches[0].layers[0], caches[1].layers[0]
    assert lyr_a.can_append_rotary(q, k, v, cos, sin)
    qa, ka, va = lyr_a.append_rotary(q, k, v, cos, sin)
    qb, kb = apply_rotary_pos_emb(q, k, cos, sin)
    kb, vb = lyr_b.update(kb, v)
    torch.cuda.synchronize()
    assert torch.equal(qa, qb) and torch.equal(ka, kb) and torch.equal(va, vb)
    assert ka.shape[2] == base + 1 and ka.is_contiguous()


@pytest.fixture
def call_log(monkeypatch):
    log = collections.Counter()
    real = _lib.call

    def spy(name, *args):
        log[name] += 1
        return real(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    yield log


def test_decoder_layer_flow_step_on_the_inplace_cache(call_log):
    """BASELINE config 5 decoder layer: prefill 3094 tokens into a
    DynamicCache, then append a 32-token flow step that attends to the whole
    prefix and to itself (non-causal, no mask) -- eager on the DynamicCache
    vs fuse_kv_rope on an InplaceKVCache (q/k norms, RoPE and append in one
    launch).  The new cache rows must be the oracle's (from the layer's own
    k projection) and the layer output equal within the GEMM tolerance (the
    attention reads strided cache views instead of contiguous tensors).
    Attention is held to the flash / memory-efficient SDPA kernels: an
    unsupported case raises rather than running the bf16 math path."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from transformers.cache_utils import DynamicCache

    layer, rot = qwen3_decoder_layer(DEV)
    P, N = 3094, 32
    torch.manual_seed(9)
    h0 = torch.randn(1, P, 4096).to(torch.bfloat16).to(DEV)
    x = torch.randn(1, N, 4096).to(torch.bfloat16).to(DEV)
    fused_sdpa = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]
    with torch.no_grad(), sdpa_kernel(fused_sdpa):
        dyn = DynamicCache()
        layer(h0, position_embeddings=rot(h0, torch.arange(P, device=DEV)[None]),
              past_key_values=dyn)
        conv = InplaceKVCache.from_dynamic(dyn, extra_tokens=N)
        cs = rot(x, torch.arange(P, P + N, device=DEV)[None])
        ref = layer(x, position_embeddings=cs, past_key_values=dyn, is_causal=False)
        assert integrate.fuse_kv_rope(layer) == 1
        out = layer(x, position_embeddings=cs, past_key_values=conv, is_causal=False)
        k_raw = layer.self_attn.k_proj(layer.input_layernorm(x)).view(1, N, -1, 128)
        torch.cuda.synchronize()
    integrate.unfuse_mlps(layer)
    # q_norm, k_norm, RoPE and the append: one launch
    assert call_log["umic_qk_rmsnorm_rope_kv_append_bf16"] == 1
    assert call_log["umic_rope_kv_append_bf16"] == 0
    lyr = conv.layers[0]
    assert lyr.get_seq_length() == P + N
    assert torch.equal(lyr.values, dyn.layers[0].values)
    assert torch.equal(lyr.keys[:, :, :P], dyn.layers[0].keys[:, :, :P])
    # the new rows are the oracle's; eager's fp32 norm statistic may round
    # across a boundary the exact one does not, one bf16 ulp at most
    kn = oracle.rmsnorm(bits(k_raw), bits(layer.self_attn.k_norm.weight),
                        layer.self_attn.k_norm.variance_epsilon)
    krot = oracle.rope_text(kn[0], bits(cs[0])[0], bits(cs[1])[0])
    assert np.array_equal(bits(lyr.keys[:, :, P:])[0], krot.transpose(1, 0, 2))
    assert ulp(bits(lyr.keys), bits(dyn.layers[0].keys)).max() <= 1
    e1, e2 = max_rel_err(out, ref), rel_err(out, ref)
    print(f"flow step on the in-place cache: max_rel {e1:.2e} rel {e2:.2e}", flush=True)
    assert e1 <= 2e-2 and e2 <= 2e-2
