"""Oracle: the native Gated DeltaNet layer around the delta rule (test infrastructure only — see
``oracle/__init__.py``).

Restates ``GatedDeltaNet.forward`` (``Heimdall/heimdall/hibrit.py:159-184``) in fp32 on the host, with
``causal_conv`` (``Heimdall/heimdall/kernels.py:29-37``), ``l2norm`` (``hibrit.py:132-133``) and ``GatedNorm``
(``hibrit.py:118-129``); the delta rule itself is ``oracle.gdn``. The frozen projections are plain matrix products
and are passed in already applied (z = in_proj_qkv(x), a, b, zg = in_proj_z(x)), as the layer's kernels receive them.

Pins (``tests/test_oracle_gdn_layer.py``): ``causal_conv`` against ``torch.nn.functional.conv1d`` with groups = C and
left padding, and against the carried prefix (two calls == one); ``l2norm`` by unit norm and direction;
``gated_norm`` against ``torch.nn.functional.rms_norm`` and a constant-row closed form; the gates against
``softplus`` / ``sigmoid``; the layer by chunk-split invariance (prefill in pieces with the carried conv and state
caches == one call, and single-token steps == prefill).
"""
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from . import gdn


def causal_conv(x: torch.Tensor, weight: torch.Tensor, prefix: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-channel causal convolution (``kernels.py:29-37``). x [B, T, C], weight [C, K] (column K - 1 = the current
    token), prefix [B, K - 1, C] (the K - 1 rows before x) or None (zeros). fp32."""
    x = x.float()
    k, t = weight.size(-1), x.size(1)
    full = F.pad(x, (0, 0, k - 1, 0)) if prefix is None else torch.cat((prefix.float(), x), dim=1)
    w = weight.float()
    y = torch.zeros_like(x)
    for j in range(k):                      # tap j: the row j tokens back, weight column K - 1 - j
        y = y + full[:, k - 1 - j:k - 1 - j + t] * w[:, k - 1 - j]
    return y


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(sum(x^2) + eps) over the last dim (``hibrit.py:132-133``)."""
    x = x.float()
    return x * torch.rsqrt(x.square().sum(-1, keepdim=True) + eps)


def gates(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias) (``hibrit.py:176-177``). Returns (g, beta) fp32."""
    beta = torch.sigmoid(b.float())
    x = a.float() + dt_bias.float()
    sp = torch.where(x > 20, x, torch.log1p(torch.exp(torch.clamp(x, max=20))))   # softplus, threshold 20
    return -A_log.float().exp() * sp, beta


def conv_inputs(z, conv_w, prefix, a, b, A_log, dt_bias, hk: int, hv: int, d: int):
    """The layer up to the delta rule (``hibrit.py:163-177``): z [B, T, C] with C = (2 hk + hv) d. Returns q, k, v
    [B, T, hv, d] (q scaled by d^-1/2, q and k repeated over the hv / hk value heads), g, beta [B, T, hv]."""
    B, T, _ = z.shape
    zc = F.silu(causal_conv(z, conv_w, prefix))
    q, k, v = zc.split((hk * d, hk * d, hv * d), dim=-1)
    r = hv // hk
    q = l2norm(q.reshape(B, T, hk, d)).repeat_interleave(r, 2) * d ** -0.5
    k = l2norm(k.reshape(B, T, hk, d)).repeat_interleave(r, 2)
    v = v.reshape(B, T, hv, d)
    g, beta = gates(a, b, A_log, dt_bias)
    return q, k, v, g, beta


def gated_norm(o: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
               bf16_points: bool = False) -> torch.Tensor:
    """weight * RMSNorm(o) * SiLU(z) over the last dim (``hibrit.py:118-129``), fp32. ``bf16_points`` rounds where the
    reference's bf16 layer rounds: o to bf16, the normalised row, and the weight product."""
    rnd = (lambda t: t.to(torch.bfloat16).float()) if bf16_points else (lambda t: t)
    xf = rnd(o.float())
    h = rnd(xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps))
    return rnd(weight.float() * h) * F.silu(z.float())


def conv_cache(z: torch.Tensor, prefix: Optional[torch.Tensor], k: int) -> torch.Tensor:
    """The new conv cache: the last K - 1 rows of [prefix; z], zero-padded in front (``hibrit.py:166-168``)."""
    full = z if prefix is None else torch.cat((prefix.to(z.dtype), z), 1)
    return F.pad(full, (0, 0, max(0, k - 1 - full.size(1)), 0))[:, -(k - 1):]


def layer_core(z, a, b, zg, conv_w, A_log, dt_bias, norm_w, hk: int, hv: int, d: int, eps: float = 1e-6,
               cache: Optional[dict] = None, bf16_points: bool = False) -> torch.Tensor:
    """GatedDeltaNet.forward between the projections (``hibrit.py:162-183``): z [B, T, C], a, b [B, T, hv],
    zg [B, T, hv * d]. Returns the gated-norm output [B, T, hv * d] fp32; ``cache`` ("conv", "S") is read and
    updated as the reference does (one token with a state runs the single-token step)."""
    B, T, _ = z.shape
    prefix = None if cache is None else cache.get("conv")
    q, k, v, g, beta = conv_inputs(z, conv_w, prefix, a, b, A_log, dt_bias, hk, hv, d)
    if cache is not None:
        cache["conv"] = conv_cache(z, prefix, conv_w.size(-1))
    s0 = None if cache is None else cache.get("S")
    if s0 is not None and T == 1:
        o, s = gdn.delta_rule_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0], s0)
        o = o[:, None]
    else:
        o, s = gdn.delta_rule_chunked(q, k, v, g, beta, 64, s0)
    if cache is not None:
        cache["S"] = s
    out = gated_norm(o, zg.reshape(B, T, hv, d), norm_w, eps, bf16_points)
    return out.reshape(B, T, hv * d)
