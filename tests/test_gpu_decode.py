"""GPU parity of K3 (layer decode step) and of the single-token delta-rule step against the CPU oracle.

The oracle runs the reference's student semantics on the CPU with the same parameters; caches share one layout, so
an oracle-built cache is copied to the GPU and both sides then decode the same tokens. Tolerances (relative L2):
<= 1e-4 for fp32 runs, <= 2e-2 for bf16 ring runs against the fp32 oracle on the same bf16 values."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn, layer as olayer

pytestmark = pytest.mark.gpu

TOL_F32, TOL_BF16 = 1e-4, 2e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def make_core(h, hkv, dh, d, window, sinks, archival=1, seed=0):
    from heimdall_amd.hibrit import BifrostCore, CoreConfig
    torch.manual_seed(seed)
    m = BifrostCore(CoreConfig(h, hkv, dh, d))
    m.convert(window, sinks, archival)
    gen = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for lin in (m.ab, m.mix):
            lin.weight.add_(torch.randn(lin.weight.shape, generator=gen) * 0.3)
            lin.bias.add_(torch.randn(lin.bias.shape, generator=gen) * 0.3)
        m.mix.bias.fill_(0.5)
        m.fq.add_(torch.randn(m.fq.shape, generator=gen) * 0.1)
        m.fk.add_(torch.randn(m.fk.shape, generator=gen) * 0.1)
        m.mix_lse.copy_(torch.randn(h, generator=gen) * 0.3)
    return m


def make_inputs(m, b, t, seed=1, dtype=torch.float32):
    c = m.c
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(b, t, c.d, generator=gen)
    q = torch.randn(b, t, c.h, c.dh, generator=gen)
    k = torch.randn(b, t, c.hkv, c.dh, generator=gen)
    v = torch.randn(b, t, c.hkv, c.dh, generator=gen)
    qr = (q + 0.1 * torch.randn(q.shape, generator=gen)).transpose(1, 2).contiguous()
    kr = (k + 0.1 * torch.randn(k.shape, generator=gen)).transpose(1, 2).contiguous()
    return tuple(z.to(dtype) for z in (x, q, k, v, qr, kr))


def split(args, a, e):
    x, q, k, v, qr, kr = args
    return x[:, a:e], q[:, a:e], k[:, a:e], v[:, a:e], qr[:, :, a:e], kr[:, :, a:e]


def to_dev(args, dev):
    return tuple(z.to(dev) for z in args)


def compare_caches(c_ref, c_gpu, tol):
    for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta", "S", "sink_k", "sink_v"):
        if key in c_ref and c_ref[key] is not None:
            assert rel(c_gpu[key], c_ref[key]) < tol, (key, rel(c_gpu[key], c_ref[key]))
    assert torch.equal(c_gpu["ring_pos"].cpu(), c_ref["ring_pos"])


def test_gdn_step_gqa_fp32(dev):
    from heimdall_amd import kernels
    gen = torch.Generator().manual_seed(5)
    B, G, R, D = 3, 2, 3, 128
    q = torch.randn(B, G * R, D, generator=gen) * D ** -0.5
    k = F.normalize(torch.randn(B, G, D, generator=gen), dim=-1)
    v = torch.randn(B, G, D, generator=gen)
    g, beta = -torch.rand(B, G, generator=gen), torch.rand(B, G, generator=gen)
    s0 = torch.randn(B, G, D, D, generator=gen) * 0.1
    with torch.no_grad():
        o, s = kernels.gdn_step(*(z.to(dev) for z in (q, k, v, g, beta, s0)))
    rep = lambda z: z.repeat_interleave(R, 1)
    o_ref, s_ref = gdn.delta_rule_step(q.double(), rep(k).double(), rep(v).double(), rep(g).double(),
                                       rep(beta).double(), rep(s0).double())
    assert rel(o, o_ref) < TOL_F32 and rel(s, s_ref[:, ::R]) < TOL_F32


@pytest.mark.parametrize("prefill", [20, 0])
def test_decode_steps_match_oracle_fp32(dev, prefill):
    """Prefill on the oracle, move the cache to the GPU, then decode step by step on both sides (positions cross
    the window and the sinks); outputs and the whole cache must agree."""
    from heimdall_amd import hibrit
    print(f"decode fp32 B=2 H=4 G=2 D=64 W=16 S=2 prefill={prefill}", flush=True)
    m = make_core(4, 2, 64, 32, window=16, sinks=2)
    args = make_inputs(m, 2, prefill + 30, seed=3)
    c_ref = {}
    if prefill:
        with torch.no_grad():
            olayer.student(m, *split(args, 0, prefill), 0, c_ref)
    c_gpu = {k_: (v_.to(dev) if torch.is_tensor(v_) else v_) for k_, v_ in c_ref.items()}
    mg = make_core(4, 2, 64, 32, window=16, sinks=2).to(dev)
    with torch.no_grad():
        for p in range(prefill, prefill + 30):
            o_ref = olayer.student(m, *split(args, p, p + 1), p, c_ref)
            o = hibrit.student(mg, *to_dev(split(args, p, p + 1), dev), p, c_gpu)
            assert rel(o, o_ref) < TOL_F32, (p, rel(o, o_ref))
    compare_caches(c_ref, c_gpu, TOL_F32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_steps_eight_heads_per_kv_D128(dev, dtype):
    """Eight query heads per KV head (the R > 4 instance of the decode kernels), D = 128, two sequences: 40 steps from
    an empty cache (the memory switches on at the window, the ring wraps twice) against the oracle; outputs and the
    whole cache must agree (fp32 to 1e-4; bf16 activations against the fp32 oracle on the same bf16 values)."""
    from heimdall_amd import hibrit
    print(f"decode {dtype} B=2 H=16 G=2 D=128 W=16 S=2, 40 steps", flush=True)
    m = make_core(16, 2, 128, 32, window=16, sinks=2)
    mg = make_core(16, 2, 128, 32, window=16, sinks=2).to(dev)
    args = make_inputs(m, 2, 40, seed=9, dtype=dtype)
    ref_args = tuple(z.float() for z in args)
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    c_ref, c_gpu = {}, {}
    with torch.no_grad():
        for p in range(40):
            o_ref = olayer.student(m, *split(ref_args, p, p + 1), p, c_ref)
            o = hibrit.student(mg, *to_dev(split(args, p, p + 1), dev), p, c_gpu)
            assert rel(o, o_ref) < tol, (p, rel(o, o_ref))
    compare_caches(c_ref, c_gpu, tol)


def test_decode_full_size_bf16(dev):
    """B=64 sequences, H=16, G=4, D=256, W=2048 + 4 sinks, bf16 ring, fp32 state ~ N(0, 0.02), one step at a
    position far past the window (memory active, ring full)."""
    from heimdall_amd import hibrit
    print("decode bf16 B=64 H=16 G=4 D=256 W=2048 S=4", flush=True)
    B, H, G, D, W, S = 64, 16, 4, 256, 2048, 4
    m = make_core(H, G, D, 64, window=W, sinks=S)
    gen = torch.Generator().manual_seed(7)
    p = 100000
    cache = {
        "sink_k": torch.randn(B, G, S, D, generator=gen).bfloat16(),
        "sink_v": torch.randn(B, G, S, D, generator=gen).bfloat16(),
        "ring_k": torch.randn(B, G, W, D, generator=gen).bfloat16(),
        "ring_v": torch.randn(B, G, W, D, generator=gen).bfloat16(),
        "ring_km": F.normalize(torch.randn(B, W, G, D, generator=gen), dim=-1),
        "ring_g": -torch.rand(B, W, G, generator=gen) * 1e-3,
        "ring_beta": torch.sigmoid(torch.randn(B, W, G, generator=gen)),
        "ring_pos": torch.empty(W, dtype=torch.long),
        "S": torch.randn(B, G, D, D, generator=gen) * 0.02,
    }
    for pp in range(p - W, p):
        cache["ring_pos"][pp % W] = pp
    x, q, k, v, qr, kr = make_inputs(m, B, 1, seed=8)
    qr, kr, v = qr.bfloat16(), kr.bfloat16(), v.bfloat16()
    c_gpu = {k_: v_.to(dev) for k_, v_ in cache.items()}
    mg = make_core(H, G, D, 64, window=W, sinks=S).to(dev)
    with torch.no_grad():
        o_ref = olayer.student(m, x, q, k, v, qr, kr, p, cache)
        o = hibrit.student(mg, *to_dev((x, q, k, v, qr, kr), dev), p, c_gpu)
    print(f"decode full-size rel err o={rel(o, o_ref):.2e} S={rel(c_gpu['S'], cache['S']):.2e}", flush=True)
    assert rel(o, o_ref) < TOL_BF16 and rel(c_gpu["S"], cache["S"]) < TOL_BF16
    compare_caches(cache, c_gpu, TOL_BF16)
