"""Pins the oracle's window + sinks attention and its LSE against textbook forms: masked softmax through
``F.scaled_dot_product_attention`` with an explicit boolean mask built from the visibility rule, ``torch.logsumexp``
over that mask in fp64, full causal attention for positions < W (``Heimdall/tests/test_hibrit.py:155-164``) and a
closed form for identical keys."""
import math

import torch
import torch.nn.functional as F

from oracle import window as win


def _mask(t, w, s):
    """visible[p, j]: sinks j < min(s, p+1), window s <= j <= p with p - j < w (Appendix A of the layer)."""
    p = torch.arange(t)[:, None]
    j = torch.arange(t)[None, :]
    return ((j < s) & (j <= p)) | ((j >= s) & (j <= p) & (p - j < w))


def test_window_equals_masked_sdpa_and_logsumexp():
    gen = torch.Generator().manual_seed(0)
    b, G, R, t, d, w, s = 2, 2, 3, 70, 16, 8, 2
    qr = torch.randn(b, G * R, t, d, generator=gen, dtype=torch.float64)
    kr = torch.randn(b, G, t, d, generator=gen, dtype=torch.float64)
    vt = torch.randn(b, G, t, d, generator=gen, dtype=torch.float64)
    o, lse = win.window_attention_from_start(qr, kr, vt, w, s)
    mask = _mask(t, w, s)
    ref = F.scaled_dot_product_attention(qr, kr.repeat_interleave(R, 1), vt.repeat_interleave(R, 1),
                                         attn_mask=mask).transpose(1, 2)
    sc = (qr @ kr.repeat_interleave(R, 1).transpose(-1, -2)) / math.sqrt(d)
    lse_ref = torch.logsumexp(sc.masked_fill(~mask, float("-inf")), -1)
    assert (o - ref).abs().max() < 1e-12 and (lse - lse_ref).abs().max() < 1e-12


def test_within_window_equals_causal_attention():
    gen = torch.Generator().manual_seed(1)
    b, G, R, t, d, w, s = 1, 2, 2, 40, 8, 16, 2
    qr = torch.randn(b, G * R, t, d, generator=gen, dtype=torch.float64)
    kr = torch.randn(b, G, t, d, generator=gen, dtype=torch.float64)
    vt = torch.randn(b, G, t, d, generator=gen, dtype=torch.float64)
    o, _ = win.window_attention_from_start(qr, kr, vt, w, s)
    full = F.scaled_dot_product_attention(qr, kr.repeat_interleave(R, 1), vt.repeat_interleave(R, 1),
                                          is_causal=True).transpose(1, 2)
    assert (o[:, :w] - full[:, :w]).abs().max() < 1e-12
    assert (o[:, w:] - full[:, w:]).abs().max() > 1e-3


def test_identical_keys_lse_closed_form():
    """All keys equal: every visible score is the same s, so lse = s + ln(#visible) and o = mean of visible v."""
    gen = torch.Generator().manual_seed(2)
    t, d, w, s = 50, 8, 8, 3
    qr = torch.randn(1, 1, t, d, generator=gen, dtype=torch.float64)
    key = torch.randn(d, generator=gen, dtype=torch.float64)
    kr = key.expand(1, 1, t, d).contiguous()
    vt = torch.randn(1, 1, t, d, generator=gen, dtype=torch.float64)
    o, lse = win.window_attention_from_start(qr, kr, vt, w, s)
    vis = _mask(t, w, s)
    sc = (qr[0, 0] @ key) / math.sqrt(d)
    n = vis.sum(-1).double()
    assert (lse[0, 0] - (sc + n.log())).abs().max() < 1e-12
    mean_v = (vis.double() @ vt[0, 0]) / n[:, None]
    assert (o[0, :, 0] - mean_v).abs().max() < 1e-12
    assert int(vis[-1].sum()) == w + s                        # steady state: W window keys + S sinks


def test_ring_split_equals_single_call():
    """Queries split into two calls, the second seeing the first call's last W keys through the ring path, give the
    single-call result (the ring is time ordered with positions; empty slots carry -1)."""
    gen = torch.Generator().manual_seed(3)
    b, G, R, t, d, w, s = 1, 1, 2, 45, 8, 8, 2
    qr = torch.randn(b, G * R, t, d, generator=gen, dtype=torch.float64)
    kr = torch.randn(b, G, t, d, generator=gen, dtype=torch.float64)
    vt = torch.randn(b, G, t, d, generator=gen, dtype=torch.float64)
    o_full, lse_full = win.window_attention_from_start(qr, kr, vt, w, s)
    a = 30
    pos = torch.arange(a, t)
    ext_k = torch.cat((kr[:, :, a - w:a], kr[:, :, a:]), 2)
    ext_v = torch.cat((vt[:, :, a - w:a], vt[:, :, a:]), 2)
    ext_pos = torch.cat((torch.arange(a - w, a), pos))
    o, lse = win.window_attention_lse(qr[:, :, a:], ext_k, ext_v, ext_pos, kr[:, :, :s], vt[:, :, :s], pos, w, s)
    assert (o - o_full[:, a:]).abs().max() < 1e-12 and (lse - lse_full[:, :, a:]).abs().max() < 1e-12


def test_blockwise_attention_matches_causal_sdpa_and_full_window():
    """The teacher's causal attention: against torch's causal scaled_dot_product_attention with the KV heads
    repeated, and against the window oracle with a window as long as the sequence and no sinks."""
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(11)
    B, H, G, T, D = 2, 6, 2, 150, 32
    qr, kr, vt = torch.randn(B, H, T, D, generator=g), torch.randn(B, G, T, D, generator=g), torch.randn(B, G, T, D, generator=g)
    o = win.blockwise_attention(qr, kr, vt)
    rep = lambda t: t.repeat_interleave(H // G, 1)
    ref = F.scaled_dot_product_attention(qr, rep(kr), rep(vt), is_causal=True).transpose(1, 2)
    assert (o - ref).abs().max() < 1e-5
    pos = torch.arange(T)
    ow, _ = win.window_attention_lse(qr, kr, vt, pos, None, None, pos, T, 0)
    assert (o - ow).abs().max() < 1e-5
