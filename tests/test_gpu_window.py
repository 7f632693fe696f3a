"""GPU parity of K2 (bf_window_fwd: window + sink attention with per-row LSE and the fused gamma mix) against the
window oracle, called directly through the C ABI.

Cases: the cache-free call from position 0 (sinks = first tokens), a chunk that reads a wrapped ring with invalid
slots, the gamma mix against a given memory read, bf16 output, batch > 1 with the reference's strided layouts
(qr [B,H,T,D], kr [B,G,T,D], v [B,T,G,D]), head dims 64/128/256, chunk lengths that are not multiples of the
128-query tile, and production geometry (D=256, W=2048 + 4 sinks). bf16 runs are compared with the fp32 oracle on
the same bf16 values: relative L2 <= 2e-2 on the output, max |lse error| <= 2e-2 (natural-log units)."""
import math

import pytest
import torch

from oracle import window as owin

pytestmark = pytest.mark.gpu

TOL_O, TOL_LSE = 2e-2, 2e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def make_case(B, H, G, D, T, W, S, start, seed, invalid_frac=0.0, dtype=torch.bfloat16):
    """Chunk tokens at positions start .. start+T-1 and a ring holding the W positions before start (slots
    p mod W), a fraction of them marked invalid (ring_pos = -1)."""
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)
    qr = rn(B, H, T, D).to(dtype)
    kr = rn(B, G, T, D).to(dtype)
    v = rn(B, T, G, D).to(dtype)                       # reference layout [B, T, G, D]
    ring_k = rn(B, G, W, D).to(dtype)
    ring_v = rn(B, G, W, D).to(dtype)
    ring_pos = torch.full((W,), -1, dtype=torch.long)
    for p in range(max(0, start - W), start):
        ring_pos[p % W] = p
    if invalid_frac > 0:
        drop = torch.rand(W, generator=gen) < invalid_frac
        ring_pos[drop] = -1
    ns = min(S, start) if start > 0 else min(S, T)
    if start > 0:
        sink_k, sink_v = rn(B, G, ns, D).to(dtype), rn(B, G, ns, D).to(dtype)
    else:
        sink_k, sink_v = kr[:, :, :ns].contiguous(), v.transpose(1, 2)[:, :, :ns].contiguous()
    return dict(qr=qr, kr=kr, v=v, ring_k=ring_k, ring_v=ring_v, ring_pos=ring_pos, sink_k=sink_k, sink_v=sink_v,
                B=B, H=H, G=G, D=D, T=T, W=W, S=S, start=start)


def oracle(c, o_mem=None, z=None, mix_lse=None, mem_scale=None):
    B, G, W, T, start = c["B"], c["G"], c["W"], c["T"], c["start"]
    f = lambda t: t.float()
    ext_pos = torch.full((W,), -1, dtype=torch.long)
    ring_k = torch.zeros(B, G, W, c["D"])
    ring_v = torch.zeros(B, G, W, c["D"])
    for i, p in enumerate(range(start - W, start)):
        if p >= 0 and c["ring_pos"][p % W] == p:
            ext_pos[i] = p
            ring_k[:, :, i] = f(c["ring_k"][:, :, p % W])
            ring_v[:, :, i] = f(c["ring_v"][:, :, p % W])
    pos = torch.arange(start, start + T)
    ext_k = torch.cat((ring_k, f(c["kr"])), 2)
    ext_v = torch.cat((ring_v, f(c["v"]).transpose(1, 2)), 2)
    ext_pos = torch.cat((ext_pos, pos))
    ns = c["sink_k"].size(2)
    o, lse = owin.window_attention_lse(f(c["qr"]), ext_k, ext_v, ext_pos, f(c["sink_k"]) if ns else None,
                                       f(c["sink_v"]) if ns else None, pos, W, c["S"])
    if o_mem is not None:
        gam = torch.sigmoid(z + mix_lse[None, None] * (lse.transpose(1, 2) - math.log(W)))
        gam = gam * (pos >= W).float()[None, :, None]
        o = o + gam[..., None] * (mem_scale[None, None, :, None] * o_mem - o)
    return o, lse


def run(c, dev, o_dtype=torch.float32, o_mem=None, z=None, mix_lse=None, mem_scale=None, use_ring=True):
    from heimdall_amd import _lib
    from heimdall_amd._device import dtype_code, stream_ptr
    lib = _lib.load()
    d = {k: (t.to(dev) if torch.is_tensor(t) else t) for k, t in c.items()}
    qr, kr, v = d["qr"], d["kr"], d["v"]
    B, H, G, D, T = c["B"], c["H"], c["G"], c["D"], c["T"]
    ns = c["sink_k"].size(2)
    o = torch.empty(B, T, H, D, dtype=o_dtype, device=dev)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    mix = o_mem is not None
    ptr = lambda t: t.data_ptr() if t is not None else None
    md = (lambda t: t.to(dev).contiguous()) if mix else (lambda t: None)
    om, zz, ml, ms = (md(t) for t in (o_mem, z, mix_lse, mem_scale)) if mix else (None,) * 4
    st = lambda t, dims: tuple(int(t.stride(i)) for i in dims)
    _lib.check(lib.bf_window_fwd(B, G, H // G, D, T, c["W"], c["S"], c["start"], dtype_code(qr.dtype),
                                 ptr(qr), *st(qr, (0, 1, 2)), ptr(kr), *st(kr, (0, 1, 2)), ptr(v), *st(v, (0, 2, 1)),
                                 ptr(d["ring_k"]) if use_ring else None, ptr(d["ring_v"]) if use_ring else None,
                                 ptr(d["ring_pos"]) if use_ring else None,
                                 ptr(d["sink_k"]) if ns else None, ptr(d["sink_v"]) if ns else None, ns, int(mix),
                                 ptr(om), dtype_code(om.dtype) if mix else 0, ptr(zz), ptr(ml), ptr(ms), ptr(o),
                                 dtype_code(o_dtype), ptr(lse),
                                 stream_ptr(dev)), "bf_window_fwd")
    torch.cuda.synchronize()
    return o.float().cpu(), lse.cpu()


def check(c, dev, **kw):
    o, lse = run(c, dev, **kw)
    mix = {k: kw[k] for k in ("o_mem", "z", "mix_lse", "mem_scale") if k in kw}
    o_ref, lse_ref = oracle(c, **mix)
    eo, el = rel(o, o_ref), (lse - lse_ref).abs().max().item()
    print(f"  rel(o)={eo:.2e} max|dlse|={el:.2e}", flush=True)
    assert eo < TOL_O and el < TOL_LSE, (eo, el)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_from_start_bf16(dev, D):
    print(f"window bf16 from 0: B=1 H=4 G=2 D={D} T=300 W=64 S=4", flush=True)
    c = make_case(1, 4, 2, D, 300, 64, 4, 0, seed=1)
    check(c, dev, use_ring=False)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_ring_wrap_invalid_slots_bf16(dev, D):
    print(f"window bf16 ring: B=2 H=6 G=2 D={D} T=200 W=256 S=4 start=1000, 20% invalid slots", flush=True)
    c = make_case(2, 6, 2, D, 200, 256, 4, 1000, seed=2, invalid_frac=0.2)
    check(c, dev)


def test_short_chunk_within_window_bf16(dev):
    """start < W: the ring is partly empty, the chunk starts inside the first window, sinks from the cache."""
    print("window bf16 start=37 T=150 W=128 S=4 D=128", flush=True)
    c = make_case(1, 4, 1, 128, 150, 128, 4, 37, seed=3)
    check(c, dev)


def test_mix_and_bf16_output(dev):
    print("window bf16 mix + bf16 out: H=4 G=2 D=256 T=260 W=128 start=100", flush=True)
    c = make_case(1, 4, 2, 256, 260, 128, 4, 100, seed=4)
    gen = torch.Generator().manual_seed(40)
    o_mem = torch.randn(1, 260, 4, 256, generator=gen) * 0.1
    z = torch.randn(1, 260, 4, generator=gen)
    mix_lse = torch.randn(4, generator=gen) * 0.3
    mem_scale = torch.full((4,), 16.0)
    check(c, dev, o_mem=o_mem, z=z, mix_lse=mix_lse, mem_scale=mem_scale)
    check(c, dev, o_dtype=torch.bfloat16, o_mem=o_mem, z=z, mix_lse=mix_lse, mem_scale=mem_scale)
    # memory read stored as bf16 (the layer's bf16 path); the oracle mixes the same bf16-rounded values
    omb = o_mem.bfloat16()
    o, lse = run(c, dev, o_mem=omb, z=z, mix_lse=mix_lse, mem_scale=mem_scale)
    o_ref, _ = oracle(c, o_mem=omb.float(), z=z, mix_lse=mix_lse, mem_scale=mem_scale)
    assert rel(o, o_ref) < TOL_O, rel(o, o_ref)


def test_production_geometry_bf16(dev):
    print("window bf16 production: H=8 G=2 D=256 W=2048 S=4 T=2600 from 0", flush=True)
    c = make_case(1, 8, 2, 256, 2600, 2048, 4, 0, seed=5)
    check(c, dev, use_ring=False)


def test_production_geometry_ring_bf16(dev):
    print("window bf16 production ring: H=8 G=2 D=256 W=2048 S=4 T=700 start=5000", flush=True)
    c = make_case(1, 8, 2, 256, 700, 2048, 4, 5000, seed=6)
    check(c, dev)


@pytest.mark.parametrize("dtype,D,T", [(torch.bfloat16, 64, 777), (torch.bfloat16, 128, 300), (torch.bfloat16, 256, 1000),
                                       (torch.float32, 128, 500), (torch.bfloat16, 256, 4096)])
def test_teacher_causal_attention(dev, dtype, D, T):
    """motor.blockwise_attention (the teacher's causal GQA attention) on bf_window_fwd with W = T and no sinks."""
    from heimdall_amd.motor import blockwise_attention
    B, H, G = (2, 6, 2) if T < 4096 else (1, 8, 2)
    print(f"teacher causal attention {dtype} B={B} H={H} G={G} D={D} T={T}", flush=True)
    gen = torch.Generator().manual_seed(T + D)
    qr = torch.randn(B, H, T, D, generator=gen).to(dtype)
    kr = torch.randn(B, G, T, D, generator=gen).to(dtype)
    vt = torch.randn(B, G, T, D, generator=gen).to(dtype)
    o = blockwise_attention(qr.to(dev), kr.to(dev), vt.to(dev))
    torch.cuda.synchronize()
    ref = owin.blockwise_attention(qr.float(), kr.float(), vt.float())
    err = rel(o, ref)
    print(f"  rel(o)={err:.2e}", flush=True)
    assert err < (1e-4 if dtype == torch.float32 else TOL_O), err
