"""Drop-in GPU operators for the reference's numerics module (``Heimdall/heimdall/kernels.py``).

``delta_rule`` and ``delta_rule_step`` keep the reference's names, argument order, layouts and return values; the
work runs in ``libbifrost_hip.so``. Inputs must be HIP tensors (there is no CPU path in this package).
"""
from typing import Optional, Tuple

import torch

from . import _lib
from ._device import BifrostError, check, gdn_forward, require_device, require_no_grad, stream_ptr


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
    return gdn_step(q, k, v, g, beta, state)


def gdn_step(q, k, v, g, beta, state, out_state: Optional[torch.Tensor] = None):
    """GQA single-token step on ``bf_gdn_step``: q [B, G*R, Dk], k [B, G, Dk], v [B, G, Dv], g, beta [B, G],
    state [B, G, Dk, Dv]. Returns (o [B, G*R, Dv] fp32, new state fp32; ``out_state`` may be ``state`` for an
    in-place update)."""
    dev = require_device(q, k, v, g, beta, state)
    require_no_grad(q, k, v, g, beta, state)
    B, H, D = q.shape
    G = k.shape[1]
    if H % G or k.shape != (B, G, D) or v.shape != (B, G, D) or state.shape != (B, G, D, D):
        raise BifrostError("inconsistent shapes for the single-token step")
    q, k, v, g, beta = (z.float().contiguous() for z in (q, k, v, g, beta))
    s_in = state.float().contiguous()
    s_out = out_state if out_state is not None else torch.empty_like(s_in)
    o = torch.empty(B, H, D, dtype=torch.float32, device=dev)
    check(_lib.load().bf_gdn_step(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                                  s_in.data_ptr(), s_out.data_ptr(), o.data_ptr(), B, G, H // G, D, stream_ptr(dev)),
          "bf_gdn_step")
    return o, s_out


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
