"""Drop-in GPU operators for the reference training engine (``Heimdall/heimdall/motor.py``): the GQA delta rule
(``:70-102``) and the teacher's causal blockwise attention (``:41-67``)."""
from typing import Optional, Tuple

import torch

from . import _lib
from ._device import BifrostError, check, dtype_code, gdn_forward, require_device, require_no_grad, stream_ptr


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


def blockwise_attention(qr, kr, vt, qblk: int = 2048, kblk: int = 8192) -> torch.Tensor:
    """Causal full attention with GQA (``Heimdall/heimdall/motor.py:41-67``, the teacher of the conversion).

    qr [B, H, T, D] (RoPE applied), kr / vt [B, G, T, D] -> o [B, T, H, D] fp32, softmax(qr kr^T / sqrt(D)) vt over
    keys j <= i. Runs ``bf_window_fwd`` with a window as long as the sequence and no sinks (every earlier key is
    visible), so no T x T matrix is formed. ``qblk`` / ``kblk`` are accepted for interface compatibility.
    """
    dev = require_device(qr, kr, vt)
    require_no_grad(qr, kr, vt)
    B, H, T, D = qr.shape
    G = kr.shape[1]
    if H % G or kr.shape != (B, G, T, D) or vt.shape != (B, G, T, D):
        raise BifrostError(f"inconsistent shapes qr{tuple(qr.shape)} kr{tuple(kr.shape)} vt{tuple(vt.shape)}")
    cdt = torch.bfloat16 if qr.dtype == torch.bfloat16 and kr.dtype == torch.bfloat16 and vt.dtype == torch.bfloat16 \
        else torch.float32
    q, k, v = (t.to(cdt) for t in (qr, kr, vt))
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    o = torch.empty(B, T, H, D, dtype=torch.float32, device=dev)
    st = lambda t: (int(t.stride(0)), int(t.stride(1)), int(t.stride(2)))
    check(_lib.load().bf_window_fwd(B, G, H // G, D, T, T, 0, 0, dtype_code(cdt), q.data_ptr(), *st(q), k.data_ptr(),
                                    *st(k), v.data_ptr(), *st(v), None, None, None, None, None, 0, 0, None, 0, None,
                                    None, None, o.data_ptr(), _lib.DTYPE_F32, None, stream_ptr(dev)),
          "bf_window_fwd")
    return o
