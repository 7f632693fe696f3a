"""Pins for ``oracle.gdn_layer`` (the native Gated DeltaNet layer around the delta rule). The reference's own tests
hold no vectors for these functions, so each is checked against a library routine or an invariant that a plausible
mistake (a reversed tap, a missing eps, a wrong repeat order, a dropped prefix row) breaks."""
import torch
import torch.nn.functional as F

from oracle import gdn_layer as ol


def rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def test_causal_conv_matches_grouped_conv1d():
    g = torch.Generator().manual_seed(0)
    B, T, C, K = 2, 37, 24, 4
    x = torch.randn(B, T, C, generator=g)
    w = torch.randn(C, K, generator=g)
    ref = F.conv1d(x.transpose(1, 2), w[:, None, :], groups=C, padding=K - 1)[..., :T].transpose(1, 2)
    assert rel(ol.causal_conv(x, w), ref) < 1e-6
    # a reversed tap order is a different filter
    assert rel(ol.causal_conv(x, w.flip(-1)), ref) > 1e-2


def test_causal_conv_prefix_carries_across_calls():
    g = torch.Generator().manual_seed(1)
    B, T, C, K = 2, 40, 16, 4
    x = torch.randn(B, T, C, generator=g)
    w = torch.randn(C, K, generator=g)
    whole = ol.causal_conv(x, w)
    for split in (1, 2, 3, 17):
        first = ol.causal_conv(x[:, :split], w)
        prefix = ol.conv_cache(x[:, :split], None, K)
        second = ol.causal_conv(x[:, split:], w, prefix)
        assert rel(torch.cat((first, second), 1), whole) < 1e-6, split


def test_l2norm_unit_norm_and_direction():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 7, 64, generator=g) * 3
    y = ol.l2norm(x)
    assert torch.allclose(y.norm(dim=-1), torch.ones(5, 7), atol=1e-5)
    cos = (y * x).sum(-1) / (y.norm(dim=-1) * x.norm(dim=-1))
    assert torch.allclose(cos, torch.ones(5, 7), atol=1e-6)
    # eps sits inside the square root: a zero row stays zero
    assert ol.l2norm(torch.zeros(1, 8)).abs().max().item() == 0.0


def test_gates_match_library_softplus_and_sigmoid():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(3, 11, 6, generator=g) * 15      # reaches past softplus's threshold of 20
    b = torch.randn(3, 11, 6, generator=g)
    A_log = torch.randn(6, generator=g)
    dt_bias = torch.randn(6, generator=g)
    gg, beta = ol.gates(a, b, A_log, dt_bias)
    assert torch.allclose(gg, -A_log.exp() * F.softplus(a + dt_bias), rtol=1e-6, atol=1e-6)
    assert torch.allclose(beta, torch.sigmoid(b))


def test_gated_norm_matches_rms_norm_and_closed_form():
    g = torch.Generator().manual_seed(4)
    o = torch.randn(4, 9, 128, generator=g)
    z = torch.randn(4, 9, 128, generator=g)
    w = torch.randn(128, generator=g)
    ref = F.rms_norm(o, (128,), weight=w, eps=1e-6) * F.silu(z)
    assert rel(ol.gated_norm(o, z, w), ref) < 1e-6
    # a constant row c normalises to c / sqrt(c^2 + eps)
    c = 0.37
    out = ol.gated_norm(torch.full((1, 64), c), torch.full((1, 64), 2.0), torch.ones(64))
    assert torch.allclose(out, torch.full((1, 64), c / (c * c + 1e-6) ** 0.5 * 2.0 * torch.sigmoid(torch.tensor(2.0)).item()))


def test_conv_inputs_repeat_order_and_scale():
    """q and k heads are repeated to consecutive value heads (repeat_interleave), q carries d^-1/2."""
    g = torch.Generator().manual_seed(5)
    B, T, hk, hv, d, K = 1, 9, 2, 4, 16, 4
    z = torch.randn(B, T, (2 * hk + hv) * d, generator=g)
    w = torch.randn((2 * hk + hv) * d, K, generator=g)
    a, b = torch.randn(B, T, hv, generator=g), torch.randn(B, T, hv, generator=g)
    q, k, v, gg, beta = ol.conv_inputs(z, w, None, a, b, torch.zeros(hv), torch.ones(hv), hk, hv, d)
    assert torch.equal(q[:, :, 0], q[:, :, 1]) and torch.equal(q[:, :, 2], q[:, :, 3])
    assert not torch.equal(q[:, :, 1], q[:, :, 2])
    assert torch.allclose(q.norm(dim=-1), torch.full((B, T, hv), d ** -0.5), atol=1e-5)
    assert torch.allclose(k.norm(dim=-1), torch.ones(B, T, hv), atol=1e-5)
    zc = F.silu(ol.causal_conv(z, w))
    assert torch.equal(v, zc[..., 2 * hk * d:].reshape(B, T, hv, d))


def _layer_case(seed, B, T, hk, hv, d, K=4):
    g = torch.Generator().manual_seed(seed)
    C = (2 * hk + hv) * d
    return dict(z=torch.randn(B, T, C, generator=g), a=torch.randn(B, T, hv, generator=g),
                b=torch.randn(B, T, hv, generator=g), zg=torch.randn(B, T, hv * d, generator=g),
                conv_w=torch.randn(C, K, generator=g) * 0.5, A_log=torch.randn(hv, generator=g) * 0.5 - 3,
                dt_bias=torch.randn(hv, generator=g), norm_w=torch.randn(d, generator=g))


def test_layer_core_split_and_single_token_invariance():
    B, T, hk, hv, d = 2, 80, 1, 2, 16
    c = _layer_case(6, B, T, hk, hv, d)
    par = (c["conv_w"], c["A_log"], c["dt_bias"], c["norm_w"], hk, hv, d)
    whole = ol.layer_core(c["z"], c["a"], c["b"], c["zg"], *par, cache={})
    cache = {}
    outs = [ol.layer_core(c["z"][:, :50], c["a"][:, :50], c["b"][:, :50], c["zg"][:, :50], *par, cache=cache)]
    for t in range(50, 53):                     # single-token steps with the carried state
        outs.append(ol.layer_core(c["z"][:, t:t + 1], c["a"][:, t:t + 1], c["b"][:, t:t + 1], c["zg"][:, t:t + 1],
                                  *par, cache=cache))
    outs.append(ol.layer_core(c["z"][:, 53:], c["a"][:, 53:], c["b"][:, 53:], c["zg"][:, 53:], *par, cache=cache))
    assert rel(torch.cat(outs, 1), whole) < 1e-5
