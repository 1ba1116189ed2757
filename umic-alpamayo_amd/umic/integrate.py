"""Module-level fusion injection -- zero model modification.

Same contract as the reference (src/umic/integrate.py): UMIC swaps the
*forward* of matching submodules at load time.  Matching is structural
(duck-typed), never by class, so any model exposing the motifs is covered;
weights are shared (no copy, no quantisation, no value change); a module
that does not match is left untouched, so applying UMIC to a model without
the motifs is a no-op.  Patching binds an instance attribute
(``module.forward = fn.__get__(module)``): ``nn.Module.__call__`` still runs
hooks, and deleting the attribute restores the class forward.

Each replacement forward first decides whether the fused gfx950 kernel
reproduces the module on the given inputs (GPU bf16 tensors of a handled
layout; for the GEMM sites also a row count in one of the site's measured
regimes -- the tiled kernel from its TILED_MIN_ROWS_* bound (at least
FUSE_MIN_ROWS), the decode GEMV up to its GEMV_ROWS_* bound; and no
gradient to carry, since the kernels have no backward).  If not, it runs
the module's own class forward -- the original eager math on whatever
device the inputs live on, recorded by autograd as usual.

Without the kernel library (libumic_hip.so missing or unloadable) every
fuser is a no-op, as the reference's fusers are without their kernel
backend (src/umic/integrate.py:653-655, 673-675): nothing is patched, the
fuser reports 0 / False with one warning, and the model keeps its eager
forwards.  The kernel wrappers called directly still raise
UmicLibraryError.
"""

from __future__ import annotations

import logging

import torch
from torch import nn

from umic import _lib
from umic.kernels import fused_ffn, layernorm, linear, rmsnorm, rope
from umic.kernels._common import grad_needed

logger = logging.getLogger(__name__)


def _backend_ready(fuser: str) -> bool:
    """True when libumic_hip.so loads.  Otherwise the named fuser patches
    nothing and reports 0 / False (the reference's no-backend behaviour,
    src/umic/integrate.py:653-655): a patched forward would otherwise raise
    at the model's first eligible call."""
    if _lib.available():
        return True
    logger.warning("%s: kernel library unavailable (%s); nothing patched", fuser,
                   _lib.load_error())
    return False

_SILU_NAMES = ("silu", "swish")

# The reference's floor for its tiled GEMM kernels (src/umic/integrate.py:
# 27-30): below it the eager intermediates are KB-scale and the vendor library
# runs the GEMMs.  Here it stays the lower bound of every site's tiled regime
# (each site's own measured bound, TILED_MIN_ROWS_* below, is at least this);
# the fewest rows take the library's GEMV instead (GEMV_ROWS_*).  Norms and
# RoPE have no floor: one fused launch always replaces several eager ones.
FUSE_MIN_ROWS = 64

# ...except for the fewest rows, the decode steps: there the library's entry
# points run a weight-streaming GEMV kernel (up to GEMV_MAX_ROWS rows).  Per
# site, the rows where it beat hipBLASLt on the config-5 decode shapes (one
# MI355X, every launch in a HIP graph over rotating weights, GEMV time as a
# fraction of the vendor's):
#   q/k/v in one launch (N = 4096 + 1024 + 1024, K = 4096): 1-8 rows, 0.24-0.62
#   q_proj / o_proj (N = 4096, K = 4096): 1-4 rows, 0.52-0.77 (5 rows: 1.15)
#   P5 gate/up (N = 2 x 12288, K = 4096): 1-4 rows, 0.54-0.67 (5 rows: 1.16)
#   down_proj (N = 4096, K = 12288): 1-2 rows, 0.89-0.98 (3 rows: 1.22)
# Rows between a site's limit and FUSE_MIN_ROWS stay on the vendor path.
GEMV_MAX_ROWS = 8     # the library's GEMV limit; the q/k/v launch takes it all
GEMV_ROWS_LINEAR = 4  # q_proj / o_proj
GEMV_ROWS_MLP = 4     # the P5 gate/up GEMV
GEMV_ROWS_DOWN = 2    # the MLP's down projection (and its residual epilogue)


# The tiled MFMA kernels against the vendor path they replace, per site and
# row count (config-5 and ViT shapes, one MI355X, each site's launches
# captured in one HIP graph over rotating operand sets, >= 640 MB a turn;
# fused time / vendor time):
#   P5 gate/up + SiLU*mul (K = 4096, N = 2 x 12288) vs two GEMMs, silu, mul:
#     M = 64: 1.45, 256: 0.91, 512: 0.82, 1024: 0.88, 2048: 0.78, 3100: 0.82, 4096: 0.91
#   ViT fc1 + bias + tanh GELU (K = 1280, N = 5120) vs F.linear then F.gelu:
#     M = 256: 1.86, 1024: 1.36, 2048: 0.98, 4096: 1.00, 8192: 0.90, 16384: 0.91
#   down_proj linear (K = 12288, N = 4096; stream-K up to 2816 rows, then
#   the four-wave stream-K schedule to 3968):
#     M = 64: 3.71, 512: 2.01, 1024: 1.46, 2048: 1.13, 2816: 1.14, 2900: 1.03,
#     3000: 1.04, 3100: 0.89, 3300: 0.94, 3500: 1.06, 3800: 1.07, 3968: 1.05,
#     4096: 1.06
#   plain q/o_proj linear (K = N = 4096):
#     M = 64: 5.1, 256: 4.1, 1024: 2.05, 2048: 1.37, 2900: 1.06, 3000: 1.07,
#     3100: 1.00, 3300: 1.04, 3500: 1.05, 3800: 0.98, 4096: 1.10, 8192: 1.10;
#     finer, two passes on one box: 3073: 1.01 / 0.97, 3100: 1.02 / 0.99,
#     3136: 1.00 / 1.00, 3200: 1.01 / 1.01, 3264: 1.03 / 1.08, 3328: 1.07 /
#     1.13, 3700: 1.01 / 1.03, 3800: 1.07 / 1.06, 3840: 1.11 / 1.08, 3900:
#     1.04 / 0.97
# The 256 x 256 tiles leave most CUs idle below a few thousand rows, where
# hipBLASLt picks smaller tiles; from there both run at the chip's power
# cap and the vendor's kernel choice decides.  So each site takes its tiled
# kernel only where it stops losing (the reference's own rule: fuse a site
# only where measured faster, integrate.py:80-91): P5 from 256 rows, fc1 +
# GELU from 2048, down_proj in the 13-tile-row band 3072..3328 (where
# hipBLASLt's pick is slow); the plain q/o linear never (None): a tie within
# +-3% from 3073 to 3200 rows and no row count where it wins on both passes.
TILED_MIN_ROWS_MLP = 256
TILED_MIN_ROWS_GELU_MLP = 2048
TILED_MIN_ROWS_DOWN = 3072
TILED_MAX_ROWS_DOWN = 3328
TILED_MIN_ROWS_LINEAR: int | None = None


def _gemm_rows_ok(x: torch.Tensor, gemv_rows: int, tiled_min: int | None) -> bool:
    """Row count in one of a site's fused GEMM regimes: the tiled kernel from
    max(FUSE_MIN_ROWS, tiled_min) rows (never when tiled_min is None), the
    GEMV up to gemv_rows."""
    rows = _rows(x)
    if 1 <= rows <= gemv_rows:
        return True
    return tiled_min is not None and rows >= max(FUSE_MIN_ROWS, tiled_min)


def _hooked(*mods) -> bool:
    """True if calling any of mods would run forward hooks (the module's own
    or global ones): the decode paths that call kernels in place of a
    submodule's __call__ then take the module call instead, so hooks fire."""
    from torch.nn.modules import module as _m

    if _m._global_forward_hooks or _m._global_forward_pre_hooks:
        return True
    return any(m is not None and (m._forward_hooks or m._forward_pre_hooks) for m in mods)


def _linear(mod: nn.Module, x: torch.Tensor, gemv_rows: int = GEMV_ROWS_LINEAR) -> torch.Tensor:
    """mod(x) for an nn.Linear, on the library's GEMV for 1..gemv_rows rows."""
    if (isinstance(mod, nn.Linear) and 1 <= _rows(x) <= gemv_rows and not _hooked(mod)
            and linear.linear_eligible(x, mod.weight, mod.bias)
            and not grad_needed(x, mod.weight, mod.bias)):
        return linear.linear_hip(x, mod.weight, mod.bias)
    return mod(x)

# Projection sites routed to the fused linear (reference integrate.py:91).
INEFFICIENT_LINEAR_NAMES = ("q_proj", "o_proj")

# Per-site choice for the P5 MLP's down_proj, which the reference leaves on
# the vendor BLAS (integrate.py:80-90, measured a loser on Thor): on MI355X
# this library's linear beats hipBLASLt in the TILED_MIN_ROWS_DOWN ..
# TILED_MAX_ROWS_DOWN band (graph-timed, one process, the four-wave stream-K
# schedule: M = 3100 236.7 against 313.7 us, M = 3300 268.6 against 286.9),
# so the fused MLP uses it there and the vendor module for every other row
# count.
DOWN_PROJ_TILED = True

# ViT projection site list kept from the reference (integrate.py:95); not
# used by apply().
VIT_LINEAR_NAMES = ("qkv",)


def _eager(module: nn.Module, *args, **kwargs):
    """Run the module's class forward (the unpatched eager implementation)."""
    return type(module).forward(module, *args, **kwargs)


def _norm_eps(module: nn.Module) -> float:
    eps = getattr(module, "variance_epsilon", None)
    if eps is None:
        eps = getattr(module, "eps", 1e-6)
    return float(eps)


def _rows(x: torch.Tensor) -> int:
    return x.numel() // x.shape[-1] if x.dim() >= 1 and x.shape[-1] else 0


# ---------------------------------------------------------------------------
# P5: gate / up / down SiLU MLP
# ---------------------------------------------------------------------------

def _is_p5_mlp(module: nn.Module) -> bool:
    """Structural match for the gate/up/down SiLU MLP motif (pattern P5)."""
    for attr in ("gate_proj", "up_proj", "down_proj"):
        sub = getattr(module, attr, None)
        if not isinstance(sub, nn.Linear) or sub.bias is not None:
            return False
    act = getattr(module, "act_fn", None) or getattr(module, "act", None)
    act_name = type(act).__name__.lower() if act is not None else ""
    return any(s in act_name for s in _SILU_NAMES)


def _fused_mlp_forward(self: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """P5-fused replacement: silu(x@Wg)*(x@Wu) in one kernel, then down."""
    wg, wu = self.gate_proj.weight, self.up_proj.weight
    if (not _gemm_rows_ok(x, GEMV_ROWS_MLP, TILED_MIN_ROWS_MLP)
            or not fused_ffn.p5_eligible(x, wg, wu) or grad_needed(x, wg, wu)):
        return _eager(self, x)
    # nn.Linear stores [out, in]; .t() is the free [in, out] view the wrapper
    # takes -- the kernel reads the original weight memory.
    h = fused_ffn.gate_silu_mul_hip(x, wg.t(), wu.t())
    down = self.down_proj
    if _rows(h) < FUSE_MIN_ROWS:
        return _linear(down, h, GEMV_ROWS_DOWN)
    if (DOWN_PROJ_TILED and isinstance(down, nn.Linear)
            and TILED_MIN_ROWS_DOWN <= _rows(h) <= TILED_MAX_ROWS_DOWN
            and linear.linear_eligible(h, down.weight, down.bias)):
        return linear.linear_hip(h, down.weight, down.bias)
    return down(h)


def fuse_mlps(model: nn.Module, dry_run: bool = False) -> int:
    """Swap the forward of every P5-matching MLP in `model`.

    Returns:
        Number of modules matched (and patched unless dry_run).
    """
    if not _backend_ready("fuse_mlps"):
        return 0
    count = 0
    for name, module in model.named_modules():
        if _is_p5_mlp(module):
            count += 1
            if not dry_run:
                module.forward = _fused_mlp_forward.__get__(module)
                logger.info("P5 fused: %s", name)
    logger.info("fuse_mlps: %d module(s) %s", count, "matched (dry run)" if dry_run else "patched")
    return count


# ---------------------------------------------------------------------------
# q / o projections
# ---------------------------------------------------------------------------

def _patched_linear_forward(self: nn.Linear, x: torch.Tensor) -> torch.Tensor:
    """Route decode calls (and, where it wins, large-M calls) to the fused
    linear; the rest stay on the vendor BLAS."""
    if (not _gemm_rows_ok(x, GEMV_ROWS_LINEAR, TILED_MIN_ROWS_LINEAR)
            or not linear.linear_eligible(x, self.weight, self.bias)
            or grad_needed(x, self.weight, self.bias)):
        return _eager(self, x)
    return linear.linear_hip(x, self.weight, self.bias)


def fuse_linears(model: nn.Module, names: tuple[str, ...] = INEFFICIENT_LINEAR_NAMES,
                 dry_run: bool = False) -> int:
    """Swap forward of nn.Linear submodules whose attribute name matches.

    Returns:
        Number of Linear modules matched (and patched unless dry_run).
    """
    if not _backend_ready("fuse_linears"):
        return 0
    count = 0
    for name, module in model.named_modules():
        leaf = name.rsplit(".", 1)[-1]
        if leaf in names and isinstance(module, nn.Linear):
            count += 1
            if not dry_run:
                module.forward = _patched_linear_forward.__get__(module)
    logger.info("fuse_linears(%s): %d module(s) %s", names, count,
                "matched (dry run)" if dry_run else "patched")
    return count


# ---------------------------------------------------------------------------
# RMSNorm and the decoder-layer residual fusion
# ---------------------------------------------------------------------------

def _patched_rmsnorm_forward(self: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """One fused kernel replacing the eager pow/mean/rsqrt/mul/cast chain."""
    if not rmsnorm.rmsnorm_eligible(x, self.weight) or grad_needed(x, self.weight):
        return _eager(self, x)
    return rmsnorm.rmsnorm_hip(x, self.weight, _norm_eps(self))


def fuse_rmsnorms(model: nn.Module, dry_run: bool = False) -> int:
    """Swap forward of every RMSNorm-family module (duck-typed).

    Match: class name contains "rmsnorm" and a 1-D `weight` (covers the
    decoder norms, q_norm / k_norm and the final norm).

    Returns:
        Number of modules matched (and patched unless dry_run).
    """
    if not _backend_ready("fuse_rmsnorms"):
        return 0
    count = 0
    for name, module in model.named_modules():
        if "rmsnorm" not in type(module).__name__.lower():
            continue
        w = getattr(module, "weight", None)
        if not isinstance(w, torch.Tensor) or w.dim() != 1:
            continue
        count += 1
        if not dry_run:
            module.forward = _patched_rmsnorm_forward.__get__(module)
    logger.info("fuse_rmsnorms: %d module(s) %s", count,
                "matched (dry run)" if dry_run else "patched")
    return count


def _is_residual_decoder_layer(module: nn.Module) -> bool:
    """Structural match for the pre-norm attn + MLP decoder block."""
    return all(hasattr(module, a) for a in
               ("input_layernorm", "post_attention_layernorm", "self_attn", "mlp"))


def _add_rmsnorm(norm: nn.Module, x: torch.Tensor, residual: torch.Tensor):
    """(norm(residual + x), residual + x): fused when the kernel applies."""
    w = getattr(norm, "weight", None)
    if ("rmsnorm" in type(norm).__name__.lower() and isinstance(w, torch.Tensor)
            and x.shape == residual.shape and residual.dtype == x.dtype
            and rmsnorm.rmsnorm_eligible(x, w) and residual.device == x.device
            and not grad_needed(x, residual, w)):
        return rmsnorm.add_rmsnorm_hip(x, residual, w, _norm_eps(norm))
    summed = residual + x
    return norm(summed), summed


def _fused_residual_layer_forward(self, hidden_states, position_embeddings=None,
                                  attention_mask=None, position_ids=None,
                                  past_key_values=None, use_cache=False, **kwargs):
    """Decoder-layer forward with the attention-residual add fused into the
    post-attention RMSNorm: one kernel emits both the MLP input and the new
    residual stream.  The MLP residual add stays a plain add (its consumer is
    the next layer's input norm), except at decode with the P5-fused MLP,
    where it is the down projection's epilogue.  Same call signature and return value as
    the transformers decoder layer; extra keyword arguments pass through.
    """
    residual = hidden_states
    attn_kwargs = dict(attention_mask=attention_mask, position_ids=position_ids,
                       past_key_values=past_key_values, use_cache=use_cache,
                       position_embeddings=position_embeddings, **kwargs)
    if (getattr(self.self_attn.forward, "__func__", None) is _fused_kv_rope_attention_forward
            and _foldable_norm(self.input_layernorm, hidden_states)):
        # decode: the attention folds input_layernorm into its q/k/v GEMV
        hidden_states, _ = self.self_attn(hidden_states=hidden_states,
                                          pre_norm=self.input_layernorm, **attn_kwargs)
    else:
        hidden_states = self.input_layernorm(hidden_states)
        hidden_states, _ = self.self_attn(hidden_states=hidden_states, **attn_kwargs)
    out = _decode_norm_mlp_residual(self.post_attention_layernorm, self.mlp, hidden_states,
                                    residual)
    if out is not None:
        return out
    hidden_states, residual = _add_rmsnorm(self.post_attention_layernorm, hidden_states, residual)
    out = _decode_mlp_residual(self.mlp, hidden_states, residual)
    if out is not None:
        return out
    hidden_states = self.mlp(hidden_states)
    return residual + hidden_states


def _foldable_norm(norm: nn.Module, x: torch.Tensor) -> bool:
    """True if the RMSNorm module `norm` of x can be folded into the decode
    GEMV that consumes its output: an RMSNorm (class name contains
    "rmsnorm", 1-D bf16 weight) without hooks, over 1..2 rows whose eager
    reduction plan the folded norm reproduces, outside autograd."""
    w = getattr(norm, "weight", None)
    return ("rmsnorm" in type(norm).__name__.lower() and isinstance(w, torch.Tensor)
            and not _hooked(norm) and rmsnorm.rmsnorm_eligible(x, w)
            and rmsnorm.gemv_norm_ok(_rows(x), x.shape[-1]) and not grad_needed(x, w))


def _decode_norm_mlp_residual(norm: nn.Module, mlp: nn.Module, x: torch.Tensor,
                              residual: torch.Tensor):
    """The decoder layer's tail at decode -- s = residual + x, then
    s + mlp(norm(s)) -- with the add and norm folded into the P5 GEMV
    (umic_add_rmsnorm_gate_silu_mul_bf16) and the residual add into the down
    projection's epilogue: two launches.  None when the MLP is not the fused
    one or the call is not eligible (the caller then runs the unfolded
    chain)."""
    if getattr(mlp.forward, "__func__", None) is not _fused_mlp_forward:
        return None
    down = getattr(mlp, "down_proj", None)
    if _hooked(mlp, down) or not _foldable_norm(norm, x):
        return None
    wg, wu = mlp.gate_proj.weight, mlp.up_proj.weight
    if not (isinstance(down, nn.Linear) and 1 <= _rows(x) <= GEMV_ROWS_DOWN
            and fused_ffn.p5_eligible(x, wg, wu)
            and residual.shape == x.shape and residual.dtype == x.dtype
            and residual.device == x.device
            and tuple(down.weight.shape) == (x.shape[-1], wg.shape[0])
            and not grad_needed(x, residual, wg, wu, down.weight, down.bias)):
        return None
    h, summed = fused_ffn.add_rmsnorm_gate_silu_mul_hip(x, residual, norm.weight,
                                                        _norm_eps(norm), wg.t(), wu.t())
    if not linear.linear_eligible(h, down.weight, down.bias):
        return summed + down(h)
    return linear.linear_add_hip(h, down.weight, down.bias, summed)


def _decode_mlp_residual(mlp: nn.Module, x: torch.Tensor, residual: torch.Tensor):
    """residual + mlp(x) for a P5-fused MLP at decode (1..GEMV_ROWS_DOWN rows):
    the fused gate_silu_mul GEMV, then down_proj with the residual add in
    its epilogue (umic_linear_add_bf16, the eager chain's two roundings).
    None when the MLP is not the fused one or the call is not eligible."""
    if getattr(mlp.forward, "__func__", None) is not _fused_mlp_forward:
        return None
    down = getattr(mlp, "down_proj", None)
    if _hooked(mlp, down):
        return None
    wg, wu = mlp.gate_proj.weight, mlp.up_proj.weight
    if not (isinstance(down, nn.Linear) and 1 <= _rows(x) <= GEMV_ROWS_DOWN
            and fused_ffn.p5_eligible(x, wg, wu)
            and residual.dtype == x.dtype and residual.device == x.device
            and residual.shape == (*x.shape[:-1], down.weight.shape[0])
            and not grad_needed(x, residual, wg, wu, down.weight, down.bias)):
        return None
    h = fused_ffn.gate_silu_mul_hip(x, wg.t(), wu.t())
    if not linear.linear_eligible(h, down.weight, down.bias):
        return residual + down(h)
    return linear.linear_add_hip(h, down.weight, down.bias, residual)


def fuse_add_rmsnorm(model: nn.Module, dry_run: bool = False) -> int:
    """Fuse the attention-residual add into post_attention_layernorm.

    Returns:
        Number of decoder layers matched (and patched unless dry_run).
    """
    if not _backend_ready("fuse_add_rmsnorm"):
        return 0
    count = 0
    for name, module in model.named_modules():
        if not _is_residual_decoder_layer(module):
            continue
        count += 1
        if not dry_run:
            module.forward = _fused_residual_layer_forward.__get__(module)
    logger.info("fuse_add_rmsnorm: %d decoder layer(s) %s", count,
                "matched (dry run)" if dry_run else "patched")
    return count


# ---------------------------------------------------------------------------
# LayerNorm and the ViT residual fusion
# ---------------------------------------------------------------------------

def _patched_layernorm_forward(self: nn.LayerNorm, x: torch.Tensor) -> torch.Tensor:
    """One fused kernel replacing eager's LayerNorm."""
    if (not layernorm.layernorm_eligible(x, self.weight, self.bias)
            or grad_needed(x, self.weight, self.bias)):
        return _eager(self, x)
    return layernorm.layernorm_hip(x, self.weight, self.bias, self.eps)


def fuse_layernorms(model: nn.Module, dry_run: bool = False) -> int:
    """Swap forward of nn.LayerNorm modules (last-dim, affine with bias)."""
    if not _backend_ready("fuse_layernorms"):
        return 0
    count = 0
    for name, module in model.named_modules():
        if (isinstance(module, nn.LayerNorm) and len(module.normalized_shape) == 1
                and module.weight is not None and module.bias is not None):
            count += 1
            if not dry_run:
                module.forward = _patched_layernorm_forward.__get__(module)
    logger.info("fuse_layernorms: %d module(s) %s", count,
                "matched (dry run)" if dry_run else "patched")
    return count


# ---------------------------------------------------------------------------
# fc1 -> GELU -> fc2 MLPs (ViT blocks)
# ---------------------------------------------------------------------------

# fc1 / fc2 attribute aliases of GELU MLPs across ViT families
# (reference integrate.py:262-263).
_FC1_NAMES = ("fc1", "linear_fc1", "up_proj")
_FC2_NAMES = ("fc2", "linear_fc2", "down_proj")

# Probe points for _gelu_kind: where erf and tanh GELU differ by up to ~5e-4.
_GELU_PROBE = torch.linspace(-6.0, 6.0, 241, dtype=torch.float32)


def _gelu_kind(act) -> str | None:
    """Which GELU `act` computes: "gelu" (erf), "gelu_tanh" or None.

    The reference matches any module whose class name contains "gelu" and
    always applies the erf form (integrate.py:284-289, kernels/linear.py:
    83-86).  That name test also accepts QuickGELU (x * sigmoid(1.702 x)) and
    the tanh forms, whose values differ; here the activation is evaluated on
    fp32 CPU probe points and identified by its values instead (activations
    hold no parameters).  The two GELU forms differ by up to ~5e-4 on the
    probe; a module within 1e-6 of neither is not fused.
    """
    if act is None or not callable(act):
        return None
    try:
        with torch.no_grad():
            y = act(_GELU_PROBE.clone())
    except Exception:  # noqa: BLE001 -- any failure means "not a plain GELU"
        return None
    if not isinstance(y, torch.Tensor) or y.shape != _GELU_PROBE.shape:
        return None
    y = y.detach().to("cpu", torch.float32)
    for kind, approx in (("gelu", "none"), ("gelu_tanh", "tanh")):
        ref = nn.functional.gelu(_GELU_PROBE, approximate=approx)
        if (y - ref).abs().max().item() <= 1e-6:
            return kind
    return None


def _mlp_act(module: nn.Module):
    for attr in ("act_fn", "act", "activation_fn"):
        act = getattr(module, attr, None)
        if act is not None:
            return act
    return None


def _is_gelu_mlp(module: nn.Module) -> tuple[nn.Linear, nn.Linear, str] | None:
    """Structural match for fc1 -> GELU -> fc2 with no gate (reference
    integrate.py:266-289): (fc1, fc2, GELU kind) or None.

    fc1.in_features must equal fc2.out_features: a projection to another
    width (the Qwen3-VL patch merger, fc1 in 4608, fc2 out 4096) shares the
    names but is not a residual FFN block.
    """
    fc1 = next((getattr(module, n) for n in _FC1_NAMES
                if isinstance(getattr(module, n, None), nn.Linear)), None)
    fc2 = next((getattr(module, n) for n in _FC2_NAMES
                if isinstance(getattr(module, n, None), nn.Linear)), None)
    if fc1 is None or fc2 is None or hasattr(module, "gate_proj"):
        return None
    if fc1.in_features != fc2.out_features or fc2.in_features != fc1.out_features:
        return None
    kind = _gelu_kind(_mlp_act(module))
    return None if kind is None else (fc1, fc2, kind)


def _fused_gelu_mlp_forward(self: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """fc1 + bias + GELU in one kernel (no fc1 output round trip before the
    activation), then fc2 on the vendor BLAS (reference integrate.py:292-303)."""
    fc1, fc2, kind = self._umic_fc
    if (_rows(x) < max(FUSE_MIN_ROWS, TILED_MIN_ROWS_GELU_MLP)
            or not linear.linear_eligible(x, fc1.weight, fc1.bias)
            or grad_needed(x, fc1.weight, fc1.bias)):
        return _eager(self, x)
    return fc2(linear.linear_hip(x, fc1.weight, fc1.bias, act=kind))


def fuse_gelu_mlps(model: nn.Module, dry_run: bool = False) -> int:
    """Fuse fc1 + GELU for every GELU-MLP module (the ViT block motif).

    Returns:
        Number of modules matched (and patched unless dry_run).
    """
    if not _backend_ready("fuse_gelu_mlps"):
        return 0
    count = 0
    for name, module in model.named_modules():
        match = _is_gelu_mlp(module)
        if match is None:
            continue
        count += 1
        if not dry_run:
            module._umic_fc = match
            module.forward = _fused_gelu_mlp_forward.__get__(module)
            logger.info("GELU MLP fused (%s): %s", match[2], name)
    logger.info("fuse_gelu_mlps: %d module(s) %s", count,
                "matched (dry run)" if dry_run else "patched")
    return count


def _add_layernorm(norm: nn.LayerNorm, x: torch.Tensor, residual: torch.Tensor):
    """(norm(residual + x), residual + x): fused when the kernel applies."""
    if (isinstance(norm, nn.LayerNorm) and len(norm.normalized_shape) == 1
            and x.shape == residual.shape and residual.dtype == x.dtype
            and residual.device == x.device
            and layernorm.layernorm_eligible(x, norm.weight, norm.bias)
            and not grad_needed(x, residual, norm.weight, norm.bias)):
        return layernorm.add_layernorm_hip(x, residual, norm.weight, norm.bias, norm.eps)
    summed = residual + x
    return norm(summed), summed


def _is_deepstack_vision_encoder(module: nn.Module) -> bool:
    """Structural match: a grid_thw-driven ViT with deepstack taps (block list
    of pre-norm LayerNorm attn + MLP blocks, patch embed, merger, deepstack
    mergers) -- reference integrate.py:481-506."""
    blocks = getattr(module, "blocks", None)
    if not blocks or len(blocks) == 0:
        return False
    b0 = blocks[0]
    if not all(hasattr(b0, a) for a in ("norm1", "norm2", "attn", "mlp")):
        return False
    if not (isinstance(getattr(b0, "norm1", None), nn.LayerNorm)
            and isinstance(getattr(b0, "norm2", None), nn.LayerNorm)):
        return False
    merger = getattr(module, "merger", None)
    if merger is None or not all(hasattr(merger, a) for a in
                                 ("norm", "linear_fc1", "act_fn", "linear_fc2",
                                  "use_postshuffle_norm", "hidden_size")):
        return False
    return all(hasattr(module, a) for a in
               ("patch_embed", "deepstack_merger_list", "deepstack_visual_indexes",
                "rotary_pos_emb", "pos_embed"))


def _vision_constants(self: nn.Module, grid_thw: torch.Tensor):
    """grid_thw-derived inputs of the ViT forward, computed as the installed
    transformers version computes them (modeling_qwen3_vl.py:690-713 with the
    transformers.vision_utils helpers; the reference used the older
    fast_pos_embed_interpolate / rot_pos_emb methods, integrate.py:547-556)."""
    from transformers import vision_utils as vu

    interp_indices, interp_weights = vu.get_vision_interpolation_indices_and_weights(
        grid_thw, num_grid_per_side=self.num_grid_per_side, mode=self.interpolation_mode,
        align_corners=self.interpolation_align_corners,
        spatial_merge_size=self.config.spatial_merge_size)
    position_ids = vu.get_vision_position_ids(grid_thw, self.spatial_merge_size)
    cu_seqlens, max_seqlen = vu.get_vision_attention_seqlens(grid_thw, self.config)
    pos_embeds = (self.pos_embed(interp_indices) * interp_weights[:, :, None]).sum(1)
    rotary = self.rotary_pos_emb(position_ids)
    rotary = rotary.reshape(rotary.shape[0], -1)
    emb = torch.cat((rotary, rotary), dim=-1)
    return pos_embeds, (emb.cos(), emb.sin()), cu_seqlens, max_seqlen


def _fused_vision_encoder_forward(self: nn.Module, hidden_states: torch.Tensor,
                                  grid_thw: torch.Tensor, **kwargs):
    """ViT forward with a grid_thw-keyed constants cache and every eligible
    residual add fused into the LayerNorm that consumes it.

    - Constants (pos_embeds, rotary cos/sin, cu_seqlens, max_seqlen) depend
      only on grid_thw and are recomputed only when its value changes.
    - Residual-add + LayerNorm fusion intra-block (attn residual into norm2)
      and cross-block (a block's MLP residual into the next block's norm1,
      or into the merger's norm after the last block when that norm works
      per token).  Deepstack tap layers materialise the plain add, since
      their mergers read the summed stream.
    Reference: integrate.py:509-611.  The eager block order is
    h = h + attn(norm1(h)); h = h + mlp(norm2(h)) (modeling_qwen3_vl.py:
    299-306); each fused add is that same bf16 add.
    """
    if torch.is_grad_enabled() and (hidden_states.requires_grad or any(
            p.requires_grad for p in self.parameters())):
        # the cached constants are detached: with autograd live, the class
        # forward (whose submodules still take their own eager fallbacks)
        return type(self).forward(self, hidden_states, grid_thw, **kwargs)
    cache: dict = self._umic_ve_cache
    key = tuple(grid_thw.reshape(-1).tolist())
    if cache.get("key") != key:
        pos_embeds, pe, cu, mx = _vision_constants(self, grid_thw)
        cache["key"] = key
        cache["consts"] = (pos_embeds.detach(), (pe[0].detach(), pe[1].detach()), cu, mx)
    pos_embeds, position_embeddings, cu_seqlens, max_seqlen = cache["consts"]

    hidden_states = self.patch_embed(hidden_states)
    hidden_states = hidden_states + pos_embeds.to(hidden_states.dtype)
    seq_len = hidden_states.shape[0]
    hidden_states = hidden_states.reshape(seq_len, -1)

    deepstack_set = self._umic_deepstack_set
    merger = self.merger
    deepstack_features = []
    pending = None
    for layer_num, blk in enumerate(self.blocks):
        if pending is None:
            normed1 = blk.norm1(hidden_states)
        else:
            normed1, hidden_states = _add_layernorm(blk.norm1, pending, hidden_states)
            pending = None
        attn_out = blk.attn(normed1, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen,
                            position_embeddings=position_embeddings, **kwargs)
        normed2, hidden_states = _add_layernorm(blk.norm2, attn_out, hidden_states)
        mlp_out = blk.mlp(normed2)
        if layer_num in deepstack_set:
            hidden_states = hidden_states + mlp_out
            idx = list(self.deepstack_visual_indexes).index(layer_num)
            deepstack_features.append(self.deepstack_merger_list[idx](hidden_states))
        else:
            pending = mlp_out

    if pending is not None and not merger.use_postshuffle_norm:
        normed, hidden_states = _add_layernorm(merger.norm, pending, hidden_states)
        x = normed.view(-1, merger.hidden_size)
        merged = merger.linear_fc2(merger.act_fn(merger.linear_fc1(x)))
    else:
        if pending is not None:
            hidden_states = hidden_states + pending
        merged = merger(hidden_states)

    out_cls = self._umic_output_cls
    if out_cls is None:
        return merged, deepstack_features
    return out_cls(last_hidden_state=hidden_states, pooler_output=merged,
                   deepstack_features=deepstack_features)


def fuse_vision_encoder_pipeline(model: nn.Module, dry_run: bool = False) -> int:
    """Fuse the grid_thw-driven ViT forward (constants cache + residual fusion).

    Composes with fuse_layernorms / fuse_vision_rope: norm, attention and MLP
    submodules are called as ordinary submodule calls, so whatever forward
    is installed on them runs.

    Returns:
        Number of vision-encoder modules matched (and patched unless dry_run).
    """
    try:
        from transformers.models.qwen3_vl import modeling_qwen3_vl as mod
        out_cls = getattr(mod, "BaseModelOutputWithDeepstackFeatures", None)
    except ImportError:
        out_cls = None
    if not _backend_ready("fuse_vision_encoder_pipeline"):
        return 0
    count = 0
    for name, module in model.named_modules():
        if not _is_deepstack_vision_encoder(module):
            continue
        count += 1
        if not dry_run:
            module._umic_ve_cache = {}
            module._umic_deepstack_set = set(module.deepstack_visual_indexes)
            module._umic_output_cls = out_cls
            module.forward = _fused_vision_encoder_forward.__get__(module)
            logger.info("vision encoder pipeline fused: %s", name)
    logger.info("fuse_vision_encoder_pipeline: %d module(s) %s", count,
                "matched (dry run)" if dry_run else "patched")
    return count


# ---------------------------------------------------------------------------
# RoPE (library-function swap in transformers' qwen3_vl module)
# ---------------------------------------------------------------------------

_ROPE_ORIGINALS: dict[str, object] = {}


def _qwen3_vl_module():
    try:
        import transformers.models.qwen3_vl.modeling_qwen3_vl as mod
    except ImportError:
        return None
    return mod


def fuse_vision_rope() -> bool:
    """Replace HF apply_rotary_pos_emb_vision with the fused q+k kernel
    (eager fallback for inputs the kernel does not handle).  Idempotent."""
    mod = _qwen3_vl_module()
    if mod is None:
        logger.warning("fuse_vision_rope: qwen3_vl module not found")
        return False
    if not _backend_ready("fuse_vision_rope"):
        return False
    cur = mod.apply_rotary_pos_emb_vision
    if getattr(cur, "_umic_fused", False):
        return True
    _ROPE_ORIGINALS.setdefault("apply_rotary_pos_emb_vision", cur)
    fused = rope.make_vision_rope(cur)
    fused._umic_fused = True
    mod.apply_rotary_pos_emb_vision = fused
    logger.info("fuse_vision_rope: apply_rotary_pos_emb_vision -> fused kernel")
    return True


def fuse_text_rope() -> bool:
    """Replace HF apply_rotary_pos_emb (text path) with the fused kernel.

    The qwen3_vl module-level function serves the LM (prefill and decode)
    and any expert built from the same text model.  Layouts the kernel does
    not handle fall back to the original function.  Idempotent.
    """
    mod = _qwen3_vl_module()
    if mod is None:
        logger.warning("fuse_text_rope: qwen3_vl module not found")
        return False
    if not _backend_ready("fuse_text_rope"):
        return False
    cur = mod.apply_rotary_pos_emb
    if getattr(cur, "_umic_fused", False):
        return True
    _ROPE_ORIGINALS.setdefault("apply_rotary_pos_emb", cur)
    fused = rope.make_text_rope(cur)
    fused._umic_fused = True
    mod.apply_rotary_pos_emb = fused
    logger.info("fuse_text_rope: apply_rotary_pos_emb -> fused kernel")
    return True


def unfuse_rope() -> int:
    """Restore the original transformers RoPE functions; returns how many."""
    mod = _qwen3_vl_module()
    if mod is None:
        return 0
    n = 0
    for name, fn in list(_ROPE_ORIGINALS.items()):
        if getattr(getattr(mod, name), "_umic_fused", False):
            setattr(mod, name, fn)
            n += 1
        del _ROPE_ORIGINALS[name]
    return n


# ---------------------------------------------------------------------------
# In-place KV cache: RoPE fused into the cache append
# ---------------------------------------------------------------------------

def _is_text_attention(module: nn.Module) -> bool:
    """Structural match for the qwen3_vl text attention: q/k/v/o
    projections, per-head q/k RMSNorms, a layer index into the cache.  The
    class must come from the transformers qwen3_vl module, whose
    ``apply_rotary_pos_emb`` (rotate_half convention) the kernel reproduces."""
    mod = _qwen3_vl_module()
    return (mod is not None and type(module).__module__ == mod.__name__
            and all(hasattr(module, a) for a in ("q_proj", "k_proj", "v_proj", "o_proj",
                                                 "q_norm", "k_norm", "head_dim", "layer_idx",
                                                 "scaling", "config"))
            and hasattr(module.config, "_attn_implementation"))


def _attention_interface(module: nn.Module):
    """The attention function transformers would call for `module`."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    impl = module.config._attn_implementation
    eager = _qwen3_vl_module().eager_attention_forward
    if impl == "eager" or impl is None:
        return eager
    return ALL_ATTENTION_FUNCTIONS.get_interface(impl, eager)


def _qkv(attn: nn.Module, x: torch.Tensor, pre_norm: nn.Module | None = None) -> list[torch.Tensor]:
    """The attention's q/k/v projections of pre_norm(x) (of x when pre_norm is
    None): in the decode regime one GEMV launch for all three
    (umic_linear_multi_bf16), with the norm folded in when it can be
    (umic_rmsnorm_linear_multi_bf16); else the norm, then each projection on
    its own."""
    mods = (attn.q_proj, attn.k_proj, attn.v_proj)
    gemv = (1 <= _rows(x) <= GEMV_MAX_ROWS and all(isinstance(m, nn.Linear) for m in mods)
            and not _hooked(*mods)
            and all(linear.linear_eligible(x, m.weight, m.bias) for m in mods)
            and not grad_needed(x, *(m.weight for m in mods), *(m.bias for m in mods)))
    if pre_norm is not None:
        if gemv and _foldable_norm(pre_norm, x):
            return linear.rmsnorm_linear_multi_hip(x, pre_norm.weight, _norm_eps(pre_norm),
                                                   [m.weight for m in mods],
                                                   [m.bias for m in mods])
        x = pre_norm(x)
    if gemv:
        return linear.linear_multi_hip(x, [m.weight for m in mods], [m.bias for m in mods])
    return [_linear(m, x) for m in mods]


def _head_norms(module: nn.Module, q: torch.Tensor):
    """``(q_w, k_w, eps)`` when the attention's q_norm / k_norm are RMSNorms
    (class name contains "rmsnorm", 1-D weight, one eps) that the fused
    norm + RoPE kernels take for ``q``; else None."""
    qn, kn = getattr(module, "q_norm", None), getattr(module, "k_norm", None)
    if not all("rmsnorm" in type(n).__name__.lower() for n in (qn, kn)) or _hooked(qn, kn):
        return None
    qw, kw = getattr(qn, "weight", None), getattr(kn, "weight", None)
    eps = _norm_eps(qn)
    if eps != _norm_eps(kn) or not rope.norm_weights_ok(q, qw, kw):
        return None
    return qw, kw, eps


def _fused_kv_rope_attention_forward(self, hidden_states, position_embeddings,
                                     attention_mask=None, past_key_values=None, pre_norm=None,
                                     **kwargs):
    """Text attention whose q/k norms, RoPE and KV-cache append are one launch.

    The projections, attention and output projection are the module's own
    (same order and arguments as the transformers forward, modeling_qwen3_vl
    ``Qwen3VLTextAttention.forward``).  Between them:

    * cache an ``InplaceKVCache``: q_norm, k_norm, RoPE and the append in one
      launch (``umic_qk_rmsnorm_rope_kv_append_bf16``), or RoPE and the
      append when the norms are not RMSNorms the kernel takes;
    * any other cache, or none: q_norm, k_norm and RoPE in one launch
      (``umic_qk_rmsnorm_rope_bf16``), then the cache's own ``update``;
    * otherwise the module's norms, ``apply_rotary_pos_emb`` and ``update``.

    pre_norm: the decoder layer's input norm, applied to hidden_states first
    (folded into the q/k/v GEMV at decode); the fused decoder-layer forward
    passes it.

    Training, or autograd through any weight or the input, runs the class
    forward.
    """
    from umic.cache import InplaceKVCache, InplaceLayer

    if self.training or grad_needed(hidden_states, self.q_proj.weight, self.k_proj.weight,
                                    self.v_proj.weight, getattr(self.q_norm, "weight", None),
                                    getattr(self.k_norm, "weight", None)):
        if pre_norm is not None:
            hidden_states = pre_norm(hidden_states)
        return type(self).forward(self, hidden_states, position_embeddings, attention_mask,
                                  past_key_values=past_key_values, **kwargs)
    layer = None
    if isinstance(past_key_values, InplaceKVCache) and self.layer_idx < len(
            past_key_values.layers):
        layer = past_key_values.layers[self.layer_idx]
        if not isinstance(layer, InplaceLayer):
            layer = None
    input_shape = hidden_states.shape[:-1]
    hidden_shape = (*input_shape, -1, self.head_dim)
    q_raw, k_raw, v = (t.view(hidden_shape) for t in _qkv(self, hidden_states, pre_norm))
    v = v.transpose(1, 2)
    cos, sin = position_embeddings
    q, k = q_raw.transpose(1, 2), k_raw.transpose(1, 2)
    norm = _head_norms(self, q)
    fused = None
    if norm is not None:
        if layer is not None:
            fused = layer.append_rotary(q, k, v, cos, sin, norm)
        elif rope.qk_norm_rope_eligible(q, k, cos, sin, norm[0], norm[1]):
            q, k = rope.qk_norm_rope(q, k, cos, sin, *norm)
            if past_key_values is not None:
                k, v = past_key_values.update(k, v, self.layer_idx)
            fused = (q, k, v)
    if fused is None:
        q = self.q_norm(q_raw).transpose(1, 2)
        k = self.k_norm(k_raw).transpose(1, 2)
        if layer is not None:
            fused = layer.append_rotary(q, k, v, cos, sin)
    if fused is not None:
        q, k, v = fused
    else:
        q, k = _qwen3_vl_module().apply_rotary_pos_emb(q, k, cos, sin)
        if past_key_values is not None:
            k, v = past_key_values.update(k, v, self.layer_idx)
    attn = _attention_interface(self)
    out, weights = attn(self, q, k, v, attention_mask, dropout=0.0, scaling=self.scaling,
                        **kwargs)
    out = out.reshape(*input_shape, -1).contiguous()
    return _linear(self.o_proj, out), weights


def fuse_kv_rope(model: nn.Module, dry_run: bool = False) -> int:
    """Route text attention through the fused q/k norms + RoPE (+ append).

    With an ``InplaceKVCache`` (see ``fuse_repeat_cache``) the per-head
    q_norm / k_norm, the RoPE and the cache append are one launch; with any
    other cache, or none, the norms and the RoPE are one launch followed by
    the cache's own ``update``.  Layouts or norms the kernels do not take
    run the module's own steps.

    Returns:
        Number of attention modules matched (and patched unless dry_run).
    """
    if _qwen3_vl_module() is None:
        logger.warning("fuse_kv_rope: qwen3_vl module not found")
        return 0
    if not _backend_ready("fuse_kv_rope"):
        return 0
    count = 0
    for _, module in model.named_modules():
        if not _is_text_attention(module):
            continue
        count += 1
        if not dry_run:
            module.forward = _fused_kv_rope_attention_forward.__get__(module)
    logger.info("fuse_kv_rope: %d attention module(s) %s", count,
                "matched (dry run)" if dry_run else "patched")
    return count


def fuse_repeat_cache(repeat_module: nn.Module, extra_tokens_hint: int = 64) -> None:
    """Replace per-step KV concatenation in append-then-crop loops.

    Contract of the reference (src/umic/integrate.py:715-756): after this,
    every call of `repeat_module` that passes a populated DynamicCache as
    ``past_key_values`` runs on an ``InplaceKVCache`` standing in for it --
    converted once per cache object, and cut back to that cache's length
    before each call -- so the loop's per-step concatenation and crop copy
    nothing.  The decision is ``umic.cache.CacheStandIn.resolve``; the
    forward pre-hook installed here only swaps the argument.  Idempotent.
    """
    from umic.cache import CacheStandIn

    if getattr(repeat_module, "_umic_repeat_cache_hook", None) is not None:
        return
    stand_in = CacheStandIn(extra_tokens_hint)

    def _swap_cache(module, args, kwargs):
        emb = kwargs.get("inputs_embeds")
        inplace = stand_in.resolve(kwargs.get("past_key_values"),
                                   emb.shape[1] if emb is not None else 0)
        if inplace is None:
            return None
        kwargs["past_key_values"] = inplace
        return args, kwargs

    repeat_module._umic_cache_stand_in = stand_in
    repeat_module._umic_repeat_cache_hook = repeat_module.register_forward_pre_hook(
        _swap_cache, with_kwargs=True)
    logger.info("fuse_repeat_cache: hook installed on %s", type(repeat_module).__name__)


def unfuse_mlps(model: nn.Module) -> int:
    """Restore original forwards (delete every instance forward override)."""
    count = 0
    for _, module in model.named_modules():
        if "forward" in module.__dict__:
            del module.__dict__["forward"]
            count += 1
    return count
