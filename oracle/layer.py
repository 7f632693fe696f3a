"""Oracle: the converted layer's student path (test infrastructure only).

``student`` restates ``HybridAttention._student`` (``Heimdall/heimdall/hibrit.py:363-424``) with its cache contract
(keys ``sink_k, sink_v, ring_k, ring_v, ring_km, ring_g, ring_beta, ring_pos, S``), ``mem_inputs`` restates
``_mem_inputs`` (``hibrit.py:327-334``) and ``convert_params`` the conversion init (``hibrit.py:211-240``).
``student_bruteforce`` is an independent per-token restatement of the same semantics (window, write-on-exit, read,
mix) used to pin the chunked/cached form.

The functions take a parameter holder ``m`` with the reference's attribute names: ``m.c.h, m.c.hkv, m.c.dh``,
``m.window, m.sinks, m.fq [H,D,D], m.fk [G,D,D], m.ab (Linear d->2G), m.mix (Linear d->H), m.mix_lse [H],
m.mem_scale [H], m.A_log [G], m.dt_bias [G], m.decay_mask [G]``.
"""
import math

import torch
import torch.nn.functional as F

from .gdn import delta_rule_chunked
from .window import window_attention_lse


def _f(t):
    return t.detach().to(torch.float64 if t.dtype == torch.float64 else torch.float32)


def mem_inputs(m, x, q, k, pos):
    """qm = normalize(q_h F_q,h) / sqrt(D), km = normalize(k_g F_k,g), g = -exp(A_log) softplus(a + dt_bias) mask,
    beta = sigmoid(b) [pos >= sinks] (``hibrit.py:327-334``). x [B,t,d], q [B,t,H,D], k [B,t,G,D], pos [t]."""
    dh = m.c.dh
    dt = torch.float64 if q.dtype == torch.float64 else torch.float32
    qm = F.normalize(torch.einsum("bthd,hde->bthe", q.to(dt), m.fq.to(dt)), dim=-1) * dh ** -0.5
    km = F.normalize(torch.einsum("bthd,hde->bthe", k.to(dt), m.fk.to(dt)), dim=-1)
    ab = F.linear(x.to(dt), m.ab.weight.to(dt), m.ab.bias.to(dt))
    a, bb = ab.chunk(2, dim=-1)
    g = -m.A_log.to(dt).exp() * F.softplus(a + m.dt_bias.to(dt)) * m.decay_mask.to(dt)
    beta = torch.sigmoid(bb) * (pos >= m.sinks).to(dt)[None, :, None]
    return qm, km, g, beta


def mix_logits(m, x):
    dt = torch.float64 if x.dtype == torch.float64 else torch.float32
    return F.linear(x.to(dt), m.mix.weight.to(dt), m.mix.bias.to(dt))


def student(m, x, q, k, v, qr, kr, start: int, cache, memory: bool = True):
    """Window + sinks attention, delta-rule memory written on window exit, gamma mix (``hibrit.py:363-424``).

    x [B,t,d]; q [B,t,H,D] (normed, pre-RoPE); k, v [B,t,G,D]; qr [B,H,t,D], kr [B,G,t,D] (RoPE'd).
    cache: dict mutated in place, or None. Returns o [B,t,H,D] in the compute dtype.
    """
    c = m.c
    b, t = x.shape[:2]
    w, s, r = m.window, m.sinks, c.h // c.hkv
    dt = torch.float64 if qr.dtype == torch.float64 else torch.float32
    st = cache if cache is not None else {}
    pos = torch.arange(start, start + t)
    vt = v.transpose(1, 2)
    sink_k, sink_v = st.get("sink_k"), st.get("sink_v")
    n_new = max(0, min(t, s - start))
    if n_new:
        sink_k = kr[:, :, :n_new] if sink_k is None else torch.cat((sink_k, kr[:, :, :n_new]), 2)
        sink_v = vt[:, :, :n_new] if sink_v is None else torch.cat((sink_v, vt[:, :, :n_new]), 2)
    pp = torch.arange(start - w, start)                       # positions the ring covers, oldest first
    if "ring_k" in st:
        idx = pp % w
        rk, rv, rkm = st["ring_k"][:, :, idx], st["ring_v"][:, :, idx], st["ring_km"][:, idx]
        rg, rb, valid = st["ring_g"][:, idx], st["ring_beta"][:, idx], st["ring_pos"][idx] == pp
    else:
        rk, rv = kr.new_zeros(b, c.hkv, w, c.dh), vt.new_zeros(b, c.hkv, w, c.dh)
        rkm = torch.zeros(b, w, c.hkv, c.dh, dtype=dt)
        rg, rb = torch.zeros(b, w, c.hkv, dtype=dt), torch.zeros(b, w, c.hkv, dtype=dt)
        valid = torch.zeros(w, dtype=torch.bool)
    ext_pos = torch.cat((torch.where(valid, pp, torch.full_like(pp, -1)), pos))
    o_win, lse = window_attention_lse(qr, torch.cat((rk.to(kr.dtype), kr), 2), torch.cat((rv.to(vt.dtype), vt), 2),
                                      ext_pos, sink_k, sink_v, pos, w, s)
    o = o_win
    use_mem = memory and start + t > w
    if use_mem or cache is not None:
        qm, km, g, beta = mem_inputs(m, x, q, k, pos)
    if use_mem:
        # token i - W is written before the query at position i reads: the write stream is ext[:t]
        vf = valid.to(dt)[None, :, None]
        wk = torch.cat((rkm.to(dt), km), 1)[:, :t]
        wv = torch.cat((rv.transpose(1, 2).to(dt), v.to(dt)), 1)[:, :t]
        wg = torch.cat((rg.to(dt) * vf, g), 1)[:, :t]
        wb = torch.cat((rb.to(dt) * vf, beta), 1)[:, :t]
        s0 = st.get("S")
        if t == 1:                                            # rank-1 step on the G states (hibrit.py:398-403)
            sm = torch.zeros(b, c.hkv, c.dh, c.dh, dtype=dt) if s0 is None else s0.to(dt)
            sm = sm * wg[:, 0].exp()[..., None, None]
            delta = (wv[:, 0] - torch.einsum("bgk,bgkv->bgv", wk[:, 0], sm)) * wb[:, 0, :, None]
            sm = sm + wk[:, 0, :, :, None] * delta[:, :, None, :]
            o_mem = torch.einsum("bgrk,bgkv->bgrv", qm[:, 0].reshape(b, c.hkv, r, c.dh), sm).reshape(b, 1, c.h, c.dh)
        else:
            # one state per KV head read by its R query heads, computed as the reference does on repeated heads
            rep = lambda z: z.repeat_interleave(r, 2)
            o_mem, sm = delta_rule_chunked(qm, rep(wk), rep(wv), rep(wg), rep(wb), 64,
                                           None if s0 is None else s0.to(dt).repeat_interleave(r, 1))
            sm = sm[:, ::r].contiguous()
        gamma = torch.sigmoid(mix_logits(m, x) + m.mix_lse.to(dt) * (lse.transpose(1, 2) - math.log(w)))
        gamma = gamma * (pos >= w).to(dt)[None, :, None]
        o = o_win + gamma[..., None] * (m.mem_scale.to(dt)[:, None] * o_mem - o_win)
        if cache is not None:
            cache["S"] = sm
    if cache is not None:
        if "ring_k" not in cache:
            cache.update(ring_k=rk, ring_v=rv, ring_km=rkm, ring_g=rg, ring_beta=rb,
                         ring_pos=torch.full((w,), -1, dtype=torch.long))
        n = min(t, w)
        slot = pos[-n:] % w
        cache["ring_k"][:, :, slot], cache["ring_v"][:, :, slot] = kr[:, :, -n:], vt[:, :, -n:]
        cache["ring_km"][:, slot], cache["ring_g"][:, slot] = km[:, -n:].to(cache["ring_km"].dtype), g[:, -n:]
        cache["ring_beta"][:, slot], cache["ring_pos"][slot] = beta[:, -n:], pos[-n:]
        cache["sink_k"], cache["sink_v"] = sink_k, sink_v
    return o


def student_bruteforce(m, x, q, k, v, qr, kr, memory: bool = True):
    """Per-token restatement from position 0 without a cache: for each p, the visible-key softmax (sinks + window),
    then the write of token p - W into the per-KV-head state, then the read and the mix. fp64 recommended."""
    c = m.c
    b, t = x.shape[:2]
    w, s, r, d = m.window, m.sinks, c.h // c.hkv, c.dh
    dt = torch.float64
    pos = torch.arange(t)
    qm, km, g, beta = mem_inputs(m, x.to(dt), q.to(dt), k.to(dt), pos)
    z = mix_logits(m, x.to(dt))
    S = torch.zeros(b, c.hkv, d, d, dtype=dt)
    out = torch.empty(b, t, c.h, d, dtype=dt)
    krf, vf, qrf = kr.to(dt), v.to(dt), qr.to(dt)
    for p in range(t):
        keys = [j for j in range(min(s, p + 1))] + [j for j in range(max(s, p - w + 1), p + 1)]
        kk = krf[:, :, keys]                                  # [b, G, n, d]
        vv = vf[:, keys].transpose(1, 2)                      # [b, G, n, d]
        jw = p - w
        if memory and jw >= 0:
            a = torch.exp(g[:, jw])                           # [b, G]
            S = S * a[..., None, None]
            recall = torch.einsum("bgk,bgkv->bgv", km[:, jw], S)
            delta = (vf[:, jw] - recall) * beta[:, jw][..., None]
            S = S + km[:, jw][..., :, None] * delta[..., None, :]
        for h in range(c.h):
            gi = h // r
            sc = torch.einsum("bd,bnd->bn", qrf[:, h, p], kk[:, gi]) / math.sqrt(d)
            lse = torch.logsumexp(sc, -1)
            o_win = torch.einsum("bn,bnd->bd", torch.exp(sc - lse[:, None]), vv[:, gi])
            if memory and p >= w:
                o_mem = torch.einsum("bk,bkv->bv", qm[:, p, h], S[:, gi])
                gam = torch.sigmoid(z[:, p, h] + m.mix_lse[h].to(dt) * (lse - math.log(w)))
                out[:, p, h] = o_win + gam[:, None] * (m.mem_scale[h].to(dt) * o_mem - o_win)
            else:
                out[:, p, h] = o_win
    return out


class Cfg:
    """Head geometry holder with the reference's attribute names (``HybridConfig.h/hkv/dh``)."""

    def __init__(self, h: int, hkv: int, dh: int, d: int):
        self.h, self.hkv, self.dh, self.d = h, hkv, dh, d


def convert_params(m, window: int, sinks: int, archival: int, generator=None, dtype=torch.float32):
    """Conversion init with mem_init="long" (``hibrit.py:211-240``): fq = I, fk = I, ab = 0, mix.w = 0, mix.b = -2,
    mix_lse = 0, dt ~ logU[1e-3, 1e-1], dt_bias = softplus^-1(dt), mem_scale = sqrt(D),
    half-life = logspace(log10 W, 6, G) tokens, A_log = log(ln2 / (life dt)), decay_mask[:archival] = 0.

    Writes the tensors onto ``m`` (attributes ab/mix are ``torch.nn.Linear``)."""
    c = m.c
    m.window, m.sinks = window, sinks
    m.fq = torch.eye(c.dh, dtype=dtype).repeat(c.h, 1, 1)
    m.fk = torch.eye(c.dh, dtype=dtype).repeat(c.hkv, 1, 1)
    m.ab = torch.nn.Linear(c.d, 2 * c.hkv).to(dtype)
    m.mix = torch.nn.Linear(c.d, c.h).to(dtype)
    with torch.no_grad():
        for lin in (m.ab, m.mix):
            lin.weight.zero_()
            lin.bias.zero_()
        m.mix.bias.fill_(-2.0)
    m.mix_lse = torch.zeros(c.h, dtype=dtype)
    u = torch.rand(c.hkv, generator=generator, dtype=torch.float64)
    dtv = torch.exp(math.log(1e-3) + u * (math.log(1e-1) - math.log(1e-3)))
    m.dt_bias = (dtv + torch.log(-torch.expm1(-dtv))).to(dtype)
    m.mem_scale = torch.full((c.h,), float(c.dh) ** 0.5, dtype=dtype)
    life = torch.logspace(math.log10(max(window, 2)), 6.0, c.hkv, dtype=torch.float64)
    m.A_log = (math.log(2.0) / (life * dtv)).log().to(dtype)
    mask = torch.ones(c.hkv, dtype=dtype)
    mask[:archival] = 0.0
    m.decay_mask = mask
    return m
