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
