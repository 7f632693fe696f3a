"""Oracle: gated delta rule (test infrastructure only — see ``oracle/__init__.py``).

Recurrence, per head, for tokens t = 1..T with alpha_t = exp(g_t):

    S_t = alpha_t S_{t-1} + beta_t k_t (v_t - alpha_t S_{t-1}^T k_t)^T,     o_t = S_t^T q_t

The chunked form follows the UT/WY representation used by the reference (``Heimdall/heimdall/kernels.py:94-129``):
inside a chunk of C tokens with in-chunk cumulative log-decay gc,

    decay_ij = exp(gc_i - gc_j) [i >= j],   A = strict_lower((beta k) k^T * decay),   Tm = (I + A)^-1
    u = Tm (beta v),  w = Tm (beta exp(gc) k),  v_new = u - w S,
    o = (q exp(gc)) S + (q k^T * decay) v_new,  S <- exp(gc_C) S + (k exp(gc_C - gc))^T v_new.

All functions take the reference's layouts: q, k [B, T, H, Dk], v [B, T, H, Dv], g, beta [B, T, H], state
[B, H, Dk, Dv]; outputs are (o [B, T, H, Dv], S [B, H, Dk, Dv]) in the compute dtype (fp32 unless fp64 inputs).
"""
from typing import Optional, Tuple

import torch
import torch.nn.functional as F


def unit_lower_inverse(a: torch.Tensor) -> torch.Tensor:
    """(I + A)^-1 for strictly lower-triangular A [..., C, C] by forward substitution.

    Follows ``Heimdall/heimdall/kernels.py:81-91`` (the reference uses ``solve_triangular`` with a
    forward-substitution fallback; both give the same matrix).
    """
    c = a.size(-1)
    eye = torch.eye(c, dtype=a.dtype, device=a.device)
    # row i of X = (I + A)^-1 solves X[i] = e_i - sum_{m<i} A[i, m] X[m]; rows are collected, not written in place,
    # so autograd can differentiate through the solve
    rows = []
    for i in range(c):
        row = eye[i].expand(a.shape[:-2] + (c,))
        if i:
            row = row - (a[..., i, :i, None] * torch.stack(rows, -2)).sum(-2)
        rows.append(row)
    return torch.stack(rows, -2)


def _compute_dtype(x: torch.Tensor) -> torch.dtype:
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def delta_rule_chunked(q, k, v, g, beta, chunk_size: int = 64,
                       initial_state: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Chunked gated delta rule, one state per head (``Heimdall/heimdall/kernels.py:94-129``).

    q is used as given (the reference passes it pre-scaled). T is padded to a multiple of ``chunk_size`` with
    g = beta = 0 rows, which leave the state unchanged (``kernels.py:106-109``).
    """
    dt = _compute_dtype(q)
    b, t, h, dk = k.shape
    dv = v.size(-1)
    qf, kf, vf = (z.to(dt).permute(0, 2, 1, 3) for z in (q, k, v))           # [b, h, t, d]
    gf, bf = (z.to(dt).permute(0, 2, 1) for z in (g, beta))                   # [b, h, t]
    c = chunk_size
    pad = (-t) % c
    if pad:
        qf, kf, vf = (F.pad(z, (0, 0, 0, pad)) for z in (qf, kf, vf))
        gf, bf = F.pad(gf, (0, pad)), F.pad(bf, (0, pad))
    n = (t + pad) // c
    qf, kf, vf = qf.reshape(b, h, n, c, dk), kf.reshape(b, h, n, c, dk), vf.reshape(b, h, n, c, dv)
    gc = gf.reshape(b, h, n, c).cumsum(-1)
    bf = bf.reshape(b, h, n, c)
    lower = torch.ones(c, c, dtype=torch.bool).tril()
    diff = gc[..., :, None] - gc[..., None, :]
    decay = torch.where(lower, diff, torch.zeros_like(diff)).exp() * lower          # [b,h,n,c,c]
    kb = kf * bf[..., None]
    a = (kb @ kf.transpose(-1, -2) * decay).tril(-1)
    tm = unit_lower_inverse(a)
    u = tm @ (vf * bf[..., None])
    w = tm @ (kb * gc.exp()[..., None])
    attn = qf @ kf.transpose(-1, -2) * decay
    q_dec = qf * gc.exp()[..., None]
    k_tail = kf * (gc[..., -1:] - gc).exp()[..., None]
    tail = gc[..., -1].exp()[..., None, None]
    s = (torch.zeros(b, h, dk, dv, dtype=dt) if initial_state is None else initial_state.to(dt).clone())
    out = torch.empty(b, h, n, c, dv, dtype=dt)
    for i in range(n):
        v_new = u[:, :, i] - w[:, :, i] @ s
        out[:, :, i] = q_dec[:, :, i] @ s + attn[:, :, i] @ v_new
        s = s * tail[:, :, i] + k_tail[:, :, i].transpose(-1, -2) @ v_new
    o = out.reshape(b, h, n * c, dv)[:, :, :t].permute(0, 2, 1, 3).contiguous()
    return o, s


def delta_rule_gqa(q, k, v, g, beta, chunk: int = 64,
                   state: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """GQA gated delta rule: one state per KV head, read by its R query heads (``Heimdall/heimdall/motor.py:70-102``).

    q [B, T, G, R, Dk], k [B, T, G, Dk], v [B, T, G, Dv], g/beta [B, T, G], state [B, G, Dk, Dv]
    -> (o [B, T, G, R, Dv], S [B, G, Dk, Dv]).
    The writes of a group do not depend on R, so the state evolution is the one-state-per-head rule on the G KV
    heads; each query head reads that state.
    """
    dt = _compute_dtype(q)
    b, t, G, R, dk = q.shape
    dv = v.size(-1)
    c = chunk
    qf = q.to(dt).permute(0, 2, 3, 1, 4)                                            # [b, G, R, t, dk]
    kf, vf = k.to(dt).permute(0, 2, 1, 3), v.to(dt).permute(0, 2, 1, 3)            # [b, G, t, d]
    gf, bf = g.to(dt).permute(0, 2, 1), beta.to(dt).permute(0, 2, 1)               # [b, G, t]
    pad = (-t) % c
    if pad:
        qf = F.pad(qf, (0, 0, 0, pad))
        kf, vf = F.pad(kf, (0, 0, 0, pad)), F.pad(vf, (0, 0, 0, pad))
        gf, bf = F.pad(gf, (0, pad)), F.pad(bf, (0, pad))
    n = (t + pad) // c
    qf = qf.reshape(b, G, R, n, c, dk)
    kf, vf = kf.reshape(b, G, n, c, dk), vf.reshape(b, G, n, c, dv)
    gc = gf.reshape(b, G, n, c).cumsum(-1)
    bf = bf.reshape(b, G, n, c)
    lower = torch.ones(c, c, dtype=torch.bool).tril()
    diff = gc[..., :, None] - gc[..., None, :]
    decay = torch.where(lower, diff, torch.zeros_like(diff)).exp() * lower          # [b,G,n,c,c]
    kb = kf * bf[..., None]
    tm = unit_lower_inverse((kb @ kf.transpose(-1, -2) * decay).tril(-1))
    u = tm @ (vf * bf[..., None])
    w = tm @ (kb * gc.exp()[..., None])
    attn = (qf @ kf[:, :, None].transpose(-1, -2)) * decay[:, :, None]              # [b,G,R,n,c,c]
    q_dec = qf * gc.exp()[:, :, None, :, :, None]
    k_tail = kf * (gc[..., -1:] - gc).exp()[..., None]
    tail = gc[..., -1].exp()[..., None, None]
    s = (torch.zeros(b, G, dk, dv, dtype=dt) if state is None else state.to(dt))
    outs = []
    for i in range(n):
        v_new = u[:, :, i] - w[:, :, i] @ s                                          # [b, G, c, dv]
        outs.append(q_dec[:, :, :, i] @ s[:, :, None] + attn[:, :, :, i] @ v_new[:, :, None])
        s = s * tail[:, :, i] + k_tail[:, :, i].transpose(-1, -2) @ v_new
    out = torch.stack(outs, 3) if outs else torch.zeros(b, G, R, 0, c, dv, dtype=dt)   # [b, G, R, n, c, dv]
    o = out.reshape(b, G, R, n * c, dv)[:, :, :, :t].permute(0, 3, 1, 2, 4).contiguous()
    return o, s


def delta_rule_step(q, k, v, g, beta, state) -> Tuple[torch.Tensor, torch.Tensor]:
    """One token (``Heimdall/heimdall/kernels.py:132-138``).

    q, k [B, H, Dk], v [B, H, Dv], g, beta [B, H], state [B, H, Dk, Dv] -> (o [B, H, Dv], S).
    """
    dt = _compute_dtype(state) if state.dtype == torch.float64 else _compute_dtype(q)
    q, k, v, g, beta, s = (z.to(dt) for z in (q, k, v, g, beta, state))
    s = s * g.exp()[..., None, None]
    recall = (k[..., :, None] * s).sum(-2)                                           # S^T k  [B, H, Dv]
    delta = (v - recall) * beta[..., None]
    s = s + k[..., :, None] * delta[..., None, :]
    return (q[..., :, None] * s).sum(-2), s


def delta_rule_recurrent(q, k, v, g, beta, initial_state=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Brute force: the closed-form recurrence applied token by token (the definition the chunked form must match).

    Same layouts as ``delta_rule_chunked``. Use fp64 inputs to pin the chunked form.
    """
    b, t, h, dk = k.shape
    dv = v.size(-1)
    dt = _compute_dtype(q)
    s = torch.zeros(b, h, dk, dv, dtype=dt) if initial_state is None else initial_state.to(dt).clone()
    o = torch.empty(b, t, h, dv, dtype=dt)
    for i in range(t):
        o[:, i], s = delta_rule_step(q[:, i], k[:, i], v[:, i], g[:, i], beta[:, i], s)
    return o, s


def delta_rule_varlen(q, k, v, g, beta, cu_seqlens, chunk_size: int = 64, initial_state=None):
    """Packed variable-length input: q [1, N_tok, H, Dk] etc., cu_seqlens [N + 1]; one independent call per sequence.

    The reference has no varlen path; its callers (``Heimdall/heimdall/hibrit.py:159-184``,
    ``Heimdall/heimdall/model.py:72-92``) run each sequence separately with its own initial state, which is what this
    restates. initial_state [N, H, Dk, Dv] or None (zeros). Returns (o [1, N_tok, H, Dv], S [N, H, Dk, Dv]).
    """
    cu = [int(x) for x in cu_seqlens]
    outs, states = [], []
    for n in range(len(cu) - 1):
        a, e = cu[n], cu[n + 1]
        s0 = None if initial_state is None else initial_state[n:n + 1]
        o, s = delta_rule_chunked(q[:, a:e], k[:, a:e], v[:, a:e], g[:, a:e], beta[:, a:e], chunk_size, s0)
        outs.append(o)
        states.append(s)
    return torch.cat(outs, 1), torch.cat(states, 0)


def delta_rule_gqa_grads(q, k, v, g, beta, state, do, ds=None, chunk: int = 64, dtype=torch.float64):
    """The gradients the reference's conversion training takes through ``motor.delta_rule_gqa``
    (``Heimdall/heimdall/motor.py:70-102`` inside ``seq_loss``, ``:149-193``): autograd of <o, do> + <S_final, ds>
    with respect to (q, k, v, g, beta, state), in fp64 (or ``dtype``). Returns the six gradients (state's is None
    without a state)."""
    xs = [x.detach().to(dtype).requires_grad_(True) for x in (q, k, v, g, beta)]
    s0 = state.detach().to(dtype).requires_grad_(True) if state is not None else None
    with torch.enable_grad():
        o, s = delta_rule_gqa(*xs, chunk=chunk, state=s0)
        loss = (o * do.to(dtype)).sum()
        if ds is not None:
            loss = loss + (s * ds.to(dtype)).sum()
        grads = torch.autograd.grad(loss, xs + ([s0] if s0 is not None else []))
    return tuple(grads) + ((None,) if s0 is None else ())
