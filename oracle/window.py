"""Oracle: sliding-window + sink attention with per-row log-sum-exp (test infrastructure only).

Restates ``HybridAttention._window_fp32`` (``Heimdall/heimdall/hibrit.py:341-361``). For a query at absolute
position p, the visible keys are the sinks j < min(S, p + 1) and the window keys j with S <= j <= p, p - j < W
(mask of ``hibrit.py:356``). Scores are (q . k) / sqrt(D), the LSE is the natural-log normaliser over the visible
keys, and the output is the softmax-weighted sum of V. Computed in fp32 (or fp64 for fp64 inputs) in query blocks
of W rows, as the reference does, so memory stays O(T * W).

``blockwise_attention`` restates the teacher's causal GQA attention (``Heimdall/heimdall/motor.py:41-67``).
"""
import torch


def window_attention_lse(qr, ext_k, ext_v, ext_pos, sink_k, sink_v, pos, window: int, sinks: int):
    """qr [B, H, t, D]; ext_k / ext_v [B, G, W + t, D] = [ring in time order ; new tokens]; ext_pos [W + t] (absolute
    positions, -1 = empty ring slot); sink_k / sink_v [B, G, ns, D] or None; pos [t] absolute query positions.

    Returns (o_win [B, t, H, D], lse [B, H, t]) in the compute dtype.
    """
    dt = torch.float64 if qr.dtype == torch.float64 else torch.float32
    b, h, t, d = qr.shape
    G = ext_k.size(1)
    w, s = window, sinks
    q = qr.to(dt).reshape(b, G, h // G, t, d) * d ** -0.5
    ns = 0 if sink_k is None else sink_k.size(2)
    spos = torch.arange(ns)
    outs, lses = [], []
    for o0 in range(0, t, w):
        n = min(w, t - o0)
        kb, vb, kp = ext_k[:, :, o0:o0 + n + w], ext_v[:, :, o0:o0 + n + w], ext_pos[o0:o0 + n + w]
        if ns:
            kb, vb, kp = torch.cat((sink_k, kb), 2), torch.cat((sink_v, vb), 2), torch.cat((spos, kp))
        is_sink = torch.arange(kp.numel()) < ns
        qp = pos[o0:o0 + n, None]
        visible = (kp >= 0) & (kp <= qp) & (is_sink | ((qp - kp < w) & (kp >= s)))
        sc = torch.matmul(q[:, :, :, o0:o0 + n], kb.to(dt)[:, :, None].transpose(-1, -2).contiguous())
        sc = sc.masked_fill(~visible, float("-inf"))
        lse = torch.logsumexp(sc, -1)
        p = torch.exp(sc - lse[..., None])
        outs.append(torch.matmul(p, vb.to(dt)[:, :, None]))
        lses.append(lse)
    o = torch.cat(outs, 3).reshape(b, h, t, d).transpose(1, 2).contiguous()
    return o, torch.cat(lses, 3).reshape(b, h, t)


def window_attention_from_start(qr, kr, vt, window: int, sinks: int):
    """The cache-free call from position 0 (``Heimdall/heimdall/motor.py:105-115``): empty ring, sinks = first tokens.

    qr [B, H, T, D], kr / vt [B, G, T, D].
    """
    b, G, t, d = kr.shape
    pos = torch.arange(t)
    ext_pos = torch.cat((torch.full((window,), -1, dtype=torch.long), pos))
    ext_k = torch.cat((kr.new_zeros(b, G, window, d), kr), 2)
    ext_v = torch.cat((vt.new_zeros(b, G, window, d), vt), 2)
    n = min(sinks, t)
    return window_attention_lse(qr, ext_k, ext_v, ext_pos, kr[:, :, :n] if n else None,
                                vt[:, :, :n] if n else None, pos, window, sinks)


def blockwise_attention(qr, kr, vt):
    """Causal full attention with GQA (``Heimdall/heimdall/motor.py:41-67``; the reference computes it with an
    online softmax over key blocks, which is the same function). qr [B, H, T, D], kr / vt [B, G, T, D] ->
    o [B, T, H, D] in the compute dtype."""
    dt = torch.float64 if qr.dtype == torch.float64 else torch.float32
    b, h, t, d = qr.shape
    g = kr.size(1)
    q = qr.to(dt).reshape(b, g, h // g, t, d) * d ** -0.5
    outs = []
    for q0 in range(0, t, 1024):
        q1 = min(t, q0 + 1024)
        sc = torch.matmul(q[:, :, :, q0:q1], kr.to(dt)[:, :, None, :q1].transpose(-1, -2).contiguous())
        mask = torch.arange(q1)[None, :] > torch.arange(q0, q1)[:, None]
        p = torch.softmax(sc.masked_fill(mask, float("-inf")), -1)
        outs.append(torch.matmul(p, vt.to(dt)[:, :, None, :q1]))
    return torch.cat(outs, 3).reshape(b, h, t, d).transpose(1, 2).contiguous()
