"""Drop-in GPU operators for the reference training engine (``Heimdall/heimdall/motor.py``): the GQA delta rule
(``:70-102``), the window + sink attention of ``precompute`` (``window_attention``, ``:105-115``) and the teacher's
causal blockwise attention (``:41-67``)."""
from typing import Optional, Tuple

import torch

from . import _lib
from ._device import (BifrostError, check, compute_dtype, dtype_code, gdn_forward, require_device,
                      require_no_grad, stream_ptr)


def _pad_tokens(x: torch.Tensor, T: int, pad: int) -> torch.Tensor:
    """[B, T, ...] -> [B, T + pad, ...] with zeros after the sequence (dim 1)."""
    if pad == 0:
        return x.contiguous()
    return torch.cat((x, x.new_zeros((x.shape[0], pad) + tuple(x.shape[2:]))), 1)


class _DeltaRuleGQA(torch.autograd.Function):
    """Forward: ``bf_gdn_fwd`` in fp32. Backward: ``bf_gdn_bwd`` (gradients of q, k, v, g, beta and the initial
    state, given those of o and of the final state)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, state):
        B, T, G, R, D = q.shape
        o, s = gdn_forward(q.reshape(B * T, G * R, D), k.reshape(B * T, G, D), v.reshape(B * T, G, D),
                           g.reshape(B * T, G), beta.reshape(B * T, G), num_seqs=B, initial_state=state)
        ctx.save_for_backward(q, k, v, g, beta, state)
        return o.view(B, T, G, R, D), s

    @staticmethod
    def backward(ctx, do, ds):
        q, k, v, g, beta, state = ctx.saved_tensors
        B, T, G, R, D = q.shape
        dev = q.device
        pad = (-T) % 64                              # beta = g = 0 on the padding: the state passes unchanged
        Tp = T + pad
        qp, kp, vp, gp, bp = (_pad_tokens(x.float(), T, pad) for x in (q, k, v, g, beta))
        dop = _pad_tokens(do.float() if do is not None else torch.zeros_like(q, dtype=torch.float32), T, pad)
        dsf = ds.float().contiguous() if ds is not None else None
        s0 = state.float().contiguous() if state is not None else None
        dq, dk, dv = torch.empty_like(qp), torch.empty_like(kp), torch.empty_like(vp)
        dg, dbeta = torch.empty_like(gp), torch.empty_like(bp)
        ds0 = torch.empty_like(s0) if s0 is not None else None
        lib = _lib.load()
        nbytes = _lib.ctypes.c_size_t(0)
        check(lib.bf_gdn_bwd_workspace_size(B, Tp, G, R, D, _lib.ctypes.byref(nbytes)), "bf_gdn_bwd_workspace_size")
        ws = torch.empty(nbytes.value, dtype=torch.uint8, device=dev)
        ptr = lambda x: x.data_ptr() if x is not None else None
        check(lib.bf_gdn_bwd(qp.data_ptr(), kp.data_ptr(), vp.data_ptr(), gp.data_ptr(), bp.data_ptr(), ptr(s0), 1.0,
                             dop.data_ptr(), ptr(dsf), B, Tp, G, R, D, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                             dg.data_ptr(), dbeta.data_ptr(), ptr(ds0), ws.data_ptr(), nbytes.value,
                             stream_ptr(dev)), "bf_gdn_bwd")
        cut = lambda x: x[:, :T]
        return (cut(dq).to(q.dtype), cut(dk).to(k.dtype), cut(dv).to(v.dtype), cut(dg).to(g.dtype),
                cut(dbeta).to(beta.dtype), ds0.to(state.dtype) if ds0 is not None else None)


def delta_rule_gqa(q, k, v, g, beta, chunk: int = 64,
                   state: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gated delta rule with one state per KV head, read by its R query heads.

    q [B, T, G, R, Dk], k [B, T, G, Dk], v [B, T, G, Dv], g / beta [B, T, G], state [B, G, Dk, Dv]
    -> (o [B, T, G, R, Dv] fp32, S [B, G, Dk, Dv] fp32). ``chunk`` is accepted for interface compatibility (the
    result is chunk-length invariant; the kernels use 64). Differentiable like the reference (fp32 throughout): with
    grad enabled and an input that requires it, the backward runs ``bf_gdn_bwd``.
    """
    require_device(q, k, v, g, beta, state)
    B, T, G, R, D = q.shape
    if v.shape[-1] != D:
        raise BifrostError("the kernels need Dk == Dv")
    inputs = (q, k, v, g, beta, state)
    if torch.is_grad_enabled() and any(x is not None and x.requires_grad for x in inputs):
        q, k, v, g, beta = (x.float() for x in (q, k, v, g, beta))
        state = state.float() if state is not None else None
        return _DeltaRuleGQA.apply(q, k, v, g, beta, state)
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


def window_attention(a, qr, kr, v) -> Tuple[torch.Tensor, torch.Tensor]:
    """Window + sink attention from position 0 with an empty ring, the cache-free path of ``_student``
    (``Heimdall/heimdall/motor.py:105-115``, called by ``precompute`` at ``:137``): ``a`` carries ``window`` and
    ``sinks``; qr [B, H, T, D], kr [B, G, T, D] (RoPE applied), v [B, T, G, D]. The sinks are the first min(sinks, T)
    tokens. Returns (o_win [B, T, H, D] fp32, lse [B, H, T] fp32), computed by ``bf_window_fwd`` (fp32 operands for
    fp32 / fp16 inputs, bf16 operands with fp32 softmax and accumulation for bf16 inputs)."""
    dev = require_device(qr, kr, v)
    require_no_grad(qr, kr, v)
    B, H, T, D = qr.shape
    G = kr.shape[1]
    if H % G or kr.shape != (B, G, T, D) or v.shape != (B, T, G, D):
        raise BifrostError(f"inconsistent shapes qr{tuple(qr.shape)} kr{tuple(kr.shape)} v{tuple(v.shape)}")
    cdt = compute_dtype(qr, kr, v)
    unit = lambda t: t if t.stride(-1) == 1 else t.contiguous()
    q_, k_, v_ = (unit(t.to(cdt)) for t in (qr, kr, v))
    ns = min(a.sinks, T)
    sk = k_[:, :, :ns].contiguous() if ns else None
    sv = v_.transpose(1, 2)[:, :, :ns].contiguous() if ns else None
    o = torch.empty(B, T, H, D, dtype=torch.float32, device=dev)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    st = lambda t, dims: tuple(int(t.stride(i)) for i in dims)
    ptr = lambda t: t.data_ptr() if t is not None else None
    check(_lib.load().bf_window_fwd(B, G, H // G, D, T, a.window, a.sinks, 0, dtype_code(cdt), q_.data_ptr(),
                                    *st(q_, (0, 1, 2)), k_.data_ptr(), *st(k_, (0, 1, 2)), v_.data_ptr(),
                                    *st(v_, (0, 2, 1)), None, None, None, ptr(sk), ptr(sv), ns, 0, None, 0, None, None,
                                    None, o.data_ptr(), _lib.DTYPE_F32, lse.data_ptr(), stream_ptr(dev)),
          "bf_window_fwd")
    return o, lse
