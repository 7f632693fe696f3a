"""GPU parity of K1 (chunked gated delta rule) against the CPU oracle, through the C ABI.

Tolerances (relative L2, ||x - ref|| / ||ref||, on o and the final state): <= 1e-4 for fp32 runs, <= 2e-2 for
bf16-input runs against the fp32 oracle evaluated on the same bf16-rounded inputs."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn

pytestmark = pytest.mark.gpu

TOL_F32, TOL_BF16 = 1e-4, 2e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm()).item()


def make(b, t, h, d, seed=0, g_lo=-0.1, s0_scale=0.1, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, h, d, generator=gen) * d ** -0.5
    k = F.normalize(torch.randn(b, t, h, d, generator=gen), dim=-1)
    v = torch.randn(b, t, h, d, generator=gen)
    g = torch.rand(b, t, h, generator=gen) * g_lo
    beta = torch.sigmoid(torch.randn(b, t, h, generator=gen))
    s0 = torch.randn(b, h, d, d, generator=gen) * s0_scale
    q, k, v = (z.to(dtype) for z in (q, k, v))
    return q, k, v, g, beta, s0


@pytest.mark.parametrize("d", [64, 128, 256])
def test_delta_rule_fp32(dev, d):
    from heimdall_amd import kernels
    print(f"gdn fp32 B=2 T=150 H=2 D={d}", flush=True)
    q, k, v, g, beta, s0 = make(2, 150, 2, d, seed=d)
    with torch.no_grad():
        o, s = kernels.delta_rule(*(z.to(dev) for z in (q, k, v, g, beta)), initial_state=s0.to(dev))
    o_ref, s_ref = gdn.delta_rule_chunked(*(z.double() for z in (q, k, v, g, beta)), 64, s0.double())
    assert o.dtype == torch.float32 and s.dtype == torch.float32
    assert rel(o, o_ref) < TOL_F32 and rel(s, s_ref) < TOL_F32, (rel(o, o_ref), rel(s, s_ref))


@pytest.mark.parametrize("d", [64, 128, 256])
def test_delta_rule_bf16(dev, d):
    from heimdall_amd import kernels
    print(f"gdn bf16 B=1 T=1000 H=4 D={d}", flush=True)
    q, k, v, g, beta, s0 = make(1, 1000, 4, d, seed=10 + d, g_lo=-1e-2, dtype=torch.bfloat16)
    with torch.no_grad():
        o, s = kernels.delta_rule(*(z.to(dev) for z in (q, k, v, g, beta)), initial_state=s0.to(dev))
    o_ref, s_ref = gdn.delta_rule_chunked(*(z.float() for z in (q, k, v, g, beta)), 64, s0)
    assert rel(o, o_ref) < TOL_BF16 and rel(s, s_ref) < TOL_BF16, (rel(o, o_ref), rel(s, s_ref))


def test_gqa_fp32(dev):
    from heimdall_amd import motor
    print("gdn gqa fp32 G=2 R=3 D=128 T=77", flush=True)
    gen = torch.Generator().manual_seed(3)
    B, T, G, R, D = 2, 77, 2, 3, 128
    q = torch.randn(B, T, G, R, D, generator=gen) * D ** -0.5
    k = F.normalize(torch.randn(B, T, G, D, generator=gen), dim=-1)
    v = torch.randn(B, T, G, D, generator=gen)
    g = -torch.rand(B, T, G, generator=gen) * 0.2
    beta = torch.rand(B, T, G, generator=gen)
    s0 = torch.randn(B, G, D, D, generator=gen) * 0.1
    with torch.no_grad():
        o, s = motor.delta_rule_gqa(*(z.to(dev) for z in (q, k, v, g, beta)), 64, s0.to(dev))
    o_ref, s_ref = gdn.delta_rule_gqa(*(z.double() for z in (q, k, v, g, beta)), 64, s0.double())
    assert rel(o, o_ref) < TOL_F32 and rel(s, s_ref) < TOL_F32


def test_varlen_bf16_with_empty_and_ragged(dev):
    from heimdall_amd import kernels
    lens = [37, 64, 0, 5, 200, 1]
    print(f"gdn varlen bf16 lens={lens} H=4 D=256", flush=True)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    q, k, v, g, beta, _ = make(1, cu[-1], 4, 256, seed=21, g_lo=-5e-3, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(22)
    s0 = torch.randn(len(lens), 4, 256, 256, generator=gen) * 0.02
    with torch.no_grad():
        o, s = kernels.delta_rule_varlen(*(z.to(dev) for z in (q, k, v, g, beta)),
                                         torch.tensor(cu, dtype=torch.int32, device=dev), s0.to(dev))
    o_ref, s_ref = gdn.delta_rule_varlen(*(z.float() for z in (q, k, v, g, beta)), torch.tensor(cu), 64, s0)
    assert rel(o, o_ref) < TOL_BF16 and rel(s, s_ref) < TOL_BF16
    assert rel(s[2], s0[2]) < 1e-6                        # empty sequence: final state = initial state


def test_step_fp32(dev):
    from heimdall_amd import kernels
    gen = torch.Generator().manual_seed(5)
    B, H, D = 3, 4, 64
    q, v = torch.randn(B, H, D, generator=gen), torch.randn(B, H, D, generator=gen)
    k = F.normalize(torch.randn(B, H, D, generator=gen), dim=-1)
    g, beta = -torch.rand(B, H, generator=gen), torch.rand(B, H, generator=gen)
    s0 = torch.randn(B, H, D, D, generator=gen) * 0.1
    with torch.no_grad():
        o, s = kernels.delta_rule_step(*(z.to(dev) for z in (q, k, v, g, beta, s0)))
    o_ref, s_ref = gdn.delta_rule_step(*(z.double() for z in (q, k, v, g, beta, s0)))
    assert rel(o, o_ref) < TOL_F32 and rel(s, s_ref) < TOL_F32


def test_full_size_split_and_linearity(dev):
    """At the headline size (T=32768, H=4, D=256, bf16): one call == two calls chained through the state, and the
    output is linear in (v, S0) for fixed q, k, g, beta (size-independent properties)."""
    from heimdall_amd import kernels
    print("gdn full-size properties T=32768 H=4 D=256 bf16", flush=True)
    B, T, H, D = 1, 32768, 4, 256
    gen = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16()
    k = F.normalize(torch.randn(B, T, H, D, device=dev, generator=gen), dim=-1).bfloat16()
    v1 = torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16()
    v2 = torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16()
    g = -torch.rand(B, T, H, device=dev, generator=gen) * 1e-3
    beta = torch.sigmoid(torch.randn(B, T, H, device=dev, generator=gen))
    with torch.no_grad():
        o, s = kernels.delta_rule(q, k, v1, g, beta)
        h = 20000                                          # not a chunk multiple: exercises the padded tail
        oa, sa = kernels.delta_rule(q[:, :h], k[:, :h], v1[:, :h], g[:, :h], beta[:, :h])
        ob, sb = kernels.delta_rule(q[:, h:], k[:, h:], v1[:, h:], g[:, h:], beta[:, h:], initial_state=sa)
        assert rel(torch.cat((oa, ob), 1), o) < 5e-3 and rel(sb, s) < 5e-3
        o2, s2 = kernels.delta_rule(q, k, v2, g, beta)
        vs = (v1.float() + v2.float()).bfloat16()
        o12, s12 = kernels.delta_rule(q, k, vs, g, beta)
        assert rel(o + o2, o12) < 2e-2 and rel(s + s2, s12) < 2e-2
        assert torch.isfinite(o).all() and torch.isfinite(s).all()


# Multi-segment scans: sequences cut into segments of `seg` chunks whose entry states come from the per-segment
# summaries (Phi, N) and their composition; the result must equal the single sequential scan of the oracle.
@pytest.mark.parametrize("d,seg", [(64, 1), (128, 2), (256, 1), (256, 3)])
def test_segments_fp32(dev, d, seg):
    from heimdall_amd._device import gdn_forward
    print(f"gdn segments fp32 B=2 T=700 H=2 D={d} segment_chunks={seg}", flush=True)
    q, k, v, g, beta, s0 = make(2, 700, 2, d, seed=30 + d + seg)
    N = 2 * 700
    with torch.no_grad():
        o, s = gdn_forward(*(z.to(dev).reshape(N, *z.shape[2:]) for z in (q, k, v)),
                           g.to(dev).reshape(N, 2), beta.to(dev).reshape(N, 2), num_seqs=2,
                           initial_state=s0.to(dev), segment_chunks=seg)
    o_ref, s_ref = gdn.delta_rule_chunked(*(z.double() for z in (q, k, v, g, beta)), 64, s0.double())
    eo, es = rel(o.view(2, 700, 2, d), o_ref), rel(s, s_ref)
    assert eo < TOL_F32 and es < TOL_F32, (eo, es)


@pytest.mark.parametrize("seg", [1, 2, 5])
def test_segments_bf16(dev, seg):
    from heimdall_amd._device import gdn_forward
    print(f"gdn segments bf16 B=1 T=1000 H=4 D=256 segment_chunks={seg}", flush=True)
    q, k, v, g, beta, s0 = make(1, 1000, 4, 256, seed=40 + seg, g_lo=-1e-2, dtype=torch.bfloat16)
    with torch.no_grad():
        o, s = gdn_forward(*(z.to(dev)[0] for z in (q, k, v, g, beta)), num_seqs=1, initial_state=s0.to(dev),
                           segment_chunks=seg)
    o_ref, s_ref = gdn.delta_rule_chunked(*(z.float() for z in (q, k, v, g, beta)), 64, s0)
    eo, es = rel(o[None], o_ref), rel(s, s_ref)
    assert eo < TOL_BF16 and es < TOL_BF16, (eo, es)


def test_segments_gqa_varlen_fp32(dev):
    """GQA (R = 3) over packed sequences with empty and one-token members, two-chunk segments."""
    from heimdall_amd._device import gdn_forward
    lens = [300, 0, 1, 130, 64, 257]
    print(f"gdn segments gqa varlen fp32 lens={lens} G=2 R=3 D=64 segment_chunks=2", flush=True)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    N, G, R, D = cu[-1], 2, 3, 64
    gen = torch.Generator().manual_seed(50)
    q = torch.randn(N, G * R, D, generator=gen) * D ** -0.5
    k = F.normalize(torch.randn(N, G, D, generator=gen), dim=-1)
    v = torch.randn(N, G, D, generator=gen)
    g = -torch.rand(N, G, generator=gen) * 0.05
    beta = torch.rand(N, G, generator=gen)
    s0 = torch.randn(len(lens), G, D, D, generator=gen) * 0.1
    with torch.no_grad():
        o, s = gdn_forward(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), num_seqs=len(lens),
                           cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=dev), initial_state=s0.to(dev),
                           segment_chunks=2)
    for n in range(len(lens)):
        a, b = cu[n], cu[n + 1]
        qq = q[a:b].view(1, b - a, G, R, D)
        o_ref, s_ref = gdn.delta_rule_gqa(qq.double(), k[a:b][None].double(), v[a:b][None].double(),
                                          g[a:b][None].double(), beta[a:b][None].double(), 64,
                                          s0[n:n + 1].double())
        if b > a:
            assert rel(o[a:b].view(1, b - a, G, R, D), o_ref) < TOL_F32, n
        assert rel(s[n:n + 1], s_ref) < TOL_F32, n
