"""Drop-in GPU operators for the reference's numerics module (``Heimdall/heimdall/kernels.py``).

``delta_rule`` and ``delta_rule_step`` keep the reference's names, argument order, layouts and return values; the
work runs in ``libbifrost_hip.so``. Inputs must be HIP tensors (there is no CPU path in this package).
"""
from typing import Optional, Tuple

import torch

from ._device import gdn_forward, require_device, require_no_grad


def delta_rule(q, k, v, g, beta, chunk_size: int = 64, initial_state: Optional[torch.Tensor] = None,
               backend: str = "auto") -> Tuple[torch.Tensor, torch.Tensor]:
    """Gated delta rule over [B, T, H, D] inputs (``Heimdall/heimdall/kernels.py:152-155`` ->
    ``delta_rule_reference`` ``:94-129``).

    q, k [B, T, H, Dk] (q pre-scaled, k L2-normalised), v [B, T, H, Dv], g, beta [B, T, H], initial_state
    [B, H, Dk, Dv]. Returns (o [B, T, H, Dv] fp32, S [B, H, Dk, Dv] fp32).

    The result does not depend on the chunk length (the UT/WY form is exact for any chunking), so ``chunk_size`` is
    accepted for interface compatibility and the kernels always use 64. ``backend`` is accepted and ignored.
    """
    require_device(q, k, v, g, beta, initial_state)
    require_no_grad(q, k, v, g, beta, initial_state)
    B, T, H, D = q.shape
    o, s = gdn_forward(q.reshape(B * T, H, D), k.reshape(B * T, H, D), v.reshape(B * T, H, v.shape[-1]),
                       g.reshape(B * T, H), beta.reshape(B * T, H), num_seqs=B, initial_state=initial_state)
    return o.view(B, T, H, -1), s


def delta_rule_step(q, k, v, g, beta, state) -> Tuple[torch.Tensor, torch.Tensor]:
    """One token (``Heimdall/heimdall/kernels.py:132-138``). q, k [B, H, Dk], v [B, H, Dv], g, beta [B, H],
    state [B, H, Dk, Dv] fp32. Returns (o [B, H, Dv] fp32, new state)."""
    require_device(q, k, v, g, beta, state)
    require_no_grad(q, k, v, g, beta, state)
    B, H, D = q.shape
    o, s = gdn_forward(q, k, v, g, beta, num_seqs=B, initial_state=state)
    return o, s


def delta_rule_varlen(q, k, v, g, beta, cu_seqlens, initial_state: Optional[torch.Tensor] = None,
                      scale: float = 1.0, head_group: int = 1) -> Tuple[torch.Tensor, torch.Tensor]:
    """Packed variable-length gated delta rule (the native Gated DeltaNet layer's core on packed sequences).

    q [1, N, H, Dk], k [1, N, H // head_group, Dk], v [1, N, H // head_group, Dv], g, beta [1, N, H // head_group],
    cu_seqlens [num_seqs + 1] (int32/int64), initial_state [num_seqs, H // head_group, Dk, Dv] or None (zeros).
    Every sequence is independent, as the reference's per-sequence calls are (``Heimdall/heimdall/hibrit.py:159-184``).
    Returns (o [1, N, H, Dv] fp32, S [num_seqs, H // head_group, Dk, Dv] fp32).
    """
    require_device(q, k, v, g, beta, initial_state)
    require_no_grad(q, k, v, g, beta, initial_state)
    _, N, H, D = q.shape
    num_seqs = cu_seqlens.numel() - 1
    o, s = gdn_forward(q[0], k[0], v[0], g[0], beta[0], num_seqs=num_seqs, cu_seqlens=cu_seqlens,
                       initial_state=initial_state, scale=scale)
    return o[None], s
