"""Drop-in GPU operator for the reference training engine's GQA delta rule (``Heimdall/heimdall/motor.py:70-102``)."""
from typing import Optional, Tuple

import torch

from ._device import gdn_forward, require_device, require_no_grad


def delta_rule_gqa(q, k, v, g, beta, chunk: int = 64,
                   state: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gated delta rule with one state per KV head, read by its R query heads.

    q [B, T, G, R, Dk], k [B, T, G, Dk], v [B, T, G, Dv], g / beta [B, T, G], state [B, G, Dk, Dv]
    -> (o [B, T, G, R, Dv] fp32, S [B, G, Dk, Dv] fp32). ``chunk`` is accepted for interface compatibility (the
    result is chunk-length invariant; the kernels use 64). Forward only.
    """
    require_device(q, k, v, g, beta, state)
    require_no_grad(q, k, v, g, beta, state)
    B, T, G, R, D = q.shape
    o, s = gdn_forward(q.reshape(B * T, G * R, D), k.reshape(B * T, G, D), v.reshape(B * T, G, v.shape[-1]),
                       g.reshape(B * T, G), beta.reshape(B * T, G), num_seqs=B, initial_state=state)
    return o.view(B, T, G, R, -1), s
