"""GPU parity of the delta-rule backward (``bf_gdn_bwd`` through ``heimdall_amd.motor.delta_rule_gqa``'s autograd)
against the oracle's gradients (``oracle.gdn.delta_rule_gqa_grads``: autograd of the restated reference in fp64, pinned
by finite differences and by the token recurrence).

Tolerance: relative L2 <= 1e-4 on every gradient (fp32 on the GPU, like the reference's training path)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def inputs(B, T, G, R, D, seed, with_state=True):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, G, R, D, generator=gen) * D ** -0.5
    k = F.normalize(torch.randn(B, T, G, D, generator=gen), dim=-1)
    v = torch.randn(B, T, G, D, generator=gen)
    g = -torch.rand(B, T, G, generator=gen) * 0.3
    beta = torch.rand(B, T, G, generator=gen)
    s0 = torch.randn(B, G, D, D, generator=gen) * 0.1 if with_state else None
    do = torch.randn(B, T, G, R, D, generator=gen)
    ds = torch.randn(B, G, D, D, generator=gen) * 0.1
    return q, k, v, g, beta, s0, do, ds


def gpu_grads(dev, q, k, v, g, beta, s0, do, ds):
    from heimdall_amd.motor import delta_rule_gqa
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, beta)]
    st = s0.to(dev).requires_grad_(True) if s0 is not None else None
    o, s = delta_rule_gqa(*xs, 64, st)
    outs, gouts = [o], [do.to(dev)]
    if ds is not None:
        outs.append(s)
        gouts.append(ds.to(dev))
    return torch.autograd.grad(outs, xs + ([st] if st is not None else []), gouts), o, s


@pytest.mark.parametrize("B,T,G,R,D,state,final", [
    (1, 64, 1, 1, 64, False, False),
    (2, 150, 2, 3, 64, True, True),          # T not a multiple of the chunk: padded like the reference
    (1, 256, 2, 2, 128, True, False),
    (1, 200, 4, 6, 256, True, True),         # the layer's head geometry
    (2, 128, 1, 4, 256, False, True),
])
def test_backward_matches_oracle(dev, B, T, G, R, D, state, final):
    q, k, v, g, beta, s0, do, ds = inputs(B, T, G, R, D, seed=T + D, with_state=state)
    ds = ds if final else None
    print(f"gdn bwd B={B} T={T} G={G} R={R} D={D} state={state} final={final}", flush=True)
    got, o, s = gpu_grads(dev, q, k, v, g, beta, s0, do, ds)
    want = gdn.delta_rule_gqa_grads(q, k, v, g, beta, s0, do, ds)
    names = ("dq", "dk", "dv", "dg", "dbeta", "ds0")
    for name, a, b in zip(names, got, want):
        assert rel(a, b) < TOL, (name, rel(a, b))
    o_ref, s_ref = gdn.delta_rule_gqa(q.double(), k.double(), v.double(), g.double(), beta.double(), 64,
                                      s0.double() if s0 is not None else None)
    assert rel(o, o_ref) < TOL and rel(s, s_ref) < TOL


def test_two_segments_carry_the_state_gradient(dev):
    """The training loss's segments (motor.seq_loss): the state of the first call feeds the second; gradients of a
    loss on both outputs equal those of one call over the whole sequence."""
    from heimdall_amd.motor import delta_rule_gqa
    B, T, G, R, D = 1, 320, 2, 3, 128
    q, k, v, g, beta, s0, do, _ = inputs(B, T, G, R, D, seed=5)
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, beta)]
    st = s0.to(dev).requires_grad_(True)
    cut = 192
    o1, s1 = delta_rule_gqa(*(x[:, :cut] for x in xs), 64, st)
    o2, _ = delta_rule_gqa(*(x[:, cut:] for x in xs), 64, s1)
    loss = (o1 * do[:, :cut].to(dev)).sum() + (o2 * do[:, cut:].to(dev)).sum()
    got = torch.autograd.grad(loss, xs + [st])
    want = gdn.delta_rule_gqa_grads(q, k, v, g, beta, s0, do, None)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), got, want):
        assert rel(a, b) < TOL, (name, rel(a, b))


def test_no_grad_path_unchanged(dev):
    """Without requires_grad the operator stays the forward-only kernel call, and the outputs agree with the
    differentiable path."""
    from heimdall_amd.motor import delta_rule_gqa
    q, k, v, g, beta, s0, _, _ = inputs(1, 100, 2, 2, 64, seed=6)
    with torch.no_grad():
        o0, s0_ = delta_rule_gqa(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), 64, s0.to(dev))
    xs = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, beta)]
    o1, s1 = delta_rule_gqa(*xs, 64, s0.to(dev))
    assert torch.equal(o0, o1.detach()) and torch.equal(s0_, s1.detach())
