"""Pins the oracle's gated delta rule against checks that do not restate its chunked formula:
brute-force token recurrence in fp64, chunk-size/padding invariance, GQA == repeated heads, closed forms
(pure decay, exact overwrite, T=1 step), varlen == per-sequence, and an independent third-party restatement
(transformers' Qwen3.5 torch fallback). Mirrors the reference tests ``Heimdall/tests/test_heimdall.py:125-137`` and
``Heimdall/tests/test_motor.py:28-39``."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn


def _inputs(b, t, h, d, seed=0, dtype=torch.float64, s0_scale=0.1, g_scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, h, d, generator=gen, dtype=dtype) * d ** -0.5
    k = F.normalize(torch.randn(b, t, h, d, generator=gen, dtype=dtype), dim=-1)
    v = torch.randn(b, t, h, d, generator=gen, dtype=dtype)
    g = -torch.rand(b, t, h, generator=gen, dtype=dtype) * g_scale
    beta = torch.rand(b, t, h, generator=gen, dtype=dtype)
    s0 = torch.randn(b, h, d, d, generator=gen, dtype=dtype) * s0_scale
    return q, k, v, g, beta, s0


@pytest.mark.parametrize("t,c", [(45, 16), (77, 16), (150, 64), (64, 64), (129, 32), (1, 64)])
def test_chunked_equals_recurrence_fp64(t, c):
    q, k, v, g, beta, s0 = _inputs(2, t, 2, 16, seed=t)
    o_ref, s_ref = gdn.delta_rule_recurrent(q, k, v, g, beta, s0)
    o, s = gdn.delta_rule_chunked(q, k, v, g, beta, c, s0)
    assert (o - o_ref).abs().max() < 1e-10 and (s - s_ref).abs().max() < 1e-10


def test_chunked_fp32_close_to_fp64():
    q, k, v, g, beta, s0 = _inputs(1, 300, 3, 32, seed=3)
    o64, s64 = gdn.delta_rule_recurrent(q, k, v, g, beta, s0)
    o, s = gdn.delta_rule_chunked(*(z.float() for z in (q, k, v, g, beta)), 64, s0.float())
    assert o.dtype == torch.float32
    rel = lambda a, b: ((a.double() - b).norm() / b.norm()).item()
    assert rel(o, o64) < 1e-5 and rel(s, s64) < 1e-5


def test_chunk_size_invariance():
    q, k, v, g, beta, s0 = _inputs(1, 200, 2, 16, seed=5)
    outs = [gdn.delta_rule_chunked(q, k, v, g, beta, c, s0) for c in (16, 32, 64)]
    for o, s in outs[1:]:
        assert (o - outs[0][0]).abs().max() < 1e-10 and (s - outs[0][1]).abs().max() < 1e-10


def test_gqa_equals_repeated_heads():
    gen = torch.Generator().manual_seed(0)
    B, T, G, R, D = 1, 77, 2, 3, 8
    q = torch.randn(B, T, G, R, D, generator=gen, dtype=torch.float64)
    k = F.normalize(torch.randn(B, T, G, D, generator=gen, dtype=torch.float64), dim=-1)
    v = torch.randn(B, T, G, D, generator=gen, dtype=torch.float64)
    g = -torch.rand(B, T, G, generator=gen, dtype=torch.float64)
    beta = torch.rand(B, T, G, generator=gen, dtype=torch.float64)
    s0 = torch.randn(B, G, D, D, generator=gen, dtype=torch.float64) * 0.1
    rep = lambda z: z.repeat_interleave(R, 2)
    o_ref, s_ref = gdn.delta_rule_recurrent(q.reshape(B, T, G * R, D), rep(k), rep(v), rep(g), rep(beta),
                                            s0.repeat_interleave(R, 1))
    o, s = gdn.delta_rule_gqa(q, k, v, g, beta, 16, s0)
    assert (o.reshape(B, T, G * R, D) - o_ref).abs().max() < 1e-10
    assert (s - s_ref[:, ::R]).abs().max() < 1e-10


def test_pure_decay_when_beta_zero():
    """beta = 0: no writes; S_T = exp(sum g) S0 and o_t = exp(cumsum g)_t S0^T q_t (closed form)."""
    q, k, v, g, beta, s0 = _inputs(1, 100, 2, 16, seed=7, g_scale=0.05)
    beta = torch.zeros_like(beta)
    o, s = gdn.delta_rule_chunked(q, k, v, g, beta, 64, s0)
    cg = g.cumsum(1)                                                          # [b, t, h]
    o_cf = torch.einsum("bthk,bhkv->bthv", q, s0) * cg.exp()[..., None]
    s_cf = s0 * cg[:, -1].exp()[..., None, None]
    assert (o - o_cf).abs().max() < 1e-12 and (s - s_cf).abs().max() < 1e-12


def test_exact_overwrite_orthonormal_keys():
    """g = 0, beta = 1, orthonormal keys, S0 = 0: every write is exact, so S^T k_j = v_j for every written j and
    S = sum_j k_j v_j^T."""
    d, t = 32, 20
    gen = torch.Generator().manual_seed(1)
    basis, _ = torch.linalg.qr(torch.randn(d, d, generator=gen, dtype=torch.float64))
    k = basis[:t][None, :, None]                                              # [1, t, 1, d]
    v = torch.randn(1, t, 1, d, generator=gen, dtype=torch.float64)
    q = torch.randn(1, t, 1, d, generator=gen, dtype=torch.float64)
    g, beta = torch.zeros(1, t, 1, dtype=torch.float64), torch.ones(1, t, 1, dtype=torch.float64)
    o, s = gdn.delta_rule_chunked(q, k, v, g, beta, 16)
    assert (s[0, 0].T @ k[0, :, 0].T - v[0, :, 0].T).abs().max() < 1e-12
    assert (s[0, 0] - k[0, :, 0].T @ v[0, :, 0]).abs().max() < 1e-12
    # overwriting a key replaces its value: write k_0 again with a new value
    v2 = torch.randn(1, 1, 1, d, generator=gen, dtype=torch.float64)
    _, s2 = gdn.delta_rule_chunked(q[:, :1], k[:, :1], v2, g[:, :1], beta[:, :1], 16, s)
    assert (s2[0, 0].T @ k[0, 0, 0] - v2[0, 0, 0]).abs().max() < 1e-12


def test_single_token_equals_step():
    q, k, v, g, beta, s0 = _inputs(3, 1, 4, 16, seed=9)
    o, s = gdn.delta_rule_chunked(q, k, v, g, beta, 64, s0)
    o1, s1 = gdn.delta_rule_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0], s0)
    # the step written out by hand for one head: decay, recall, delta, rank-1 write, read
    b, h = 1, 2
    S = s0[b, h] * math.exp(g[b, 0, h])
    delta = beta[b, 0, h] * (v[b, 0, h] - S.T @ k[b, 0, h])
    S = S + torch.outer(k[b, 0, h], delta)
    assert (S - s1[b, h]).abs().max() < 1e-12 and (S.T @ q[b, 0, h] - o1[b, h]).abs().max() < 1e-12
    assert (o[:, 0] - o1).abs().max() < 1e-12 and (s - s1).abs().max() < 1e-12


def test_varlen_equals_per_sequence():
    lens = [37, 64, 5, 100]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    q, k, v, g, beta, _ = _inputs(1, cu[-1], 2, 16, seed=11)
    gen = torch.Generator().manual_seed(12)
    s0 = torch.randn(len(lens), 2, 16, 16, generator=gen, dtype=torch.float64) * 0.1
    o, s = gdn.delta_rule_varlen(q, k, v, g, beta, torch.tensor(cu), 64, s0)
    for n in range(len(lens)):
        a, e = cu[n], cu[n + 1]
        o_r, s_r = gdn.delta_rule_recurrent(q[:, a:e], k[:, a:e], v[:, a:e], g[:, a:e], beta[:, a:e], s0[n:n + 1])
        assert (o[:, a:e] - o_r).abs().max() < 1e-10 and (s[n] - s_r[0]).abs().max() < 1e-10


def test_unit_lower_inverse_is_inverse():
    gen = torch.Generator().manual_seed(2)
    a = torch.randn(3, 64, 64, generator=gen, dtype=torch.float64).tril(-1) * 0.2
    inv = gdn.unit_lower_inverse(a)
    eye = torch.eye(64, dtype=torch.float64)
    assert (inv @ (eye + a) - eye).abs().max() < 1e-10
    assert torch.equal(inv.triu(1), torch.zeros_like(inv)) and torch.equal(inv.diagonal(dim1=-2, dim2=-1),
                                                                          torch.ones(3, 64, dtype=torch.float64))


def test_matches_transformers_restatement():
    """Independent third-party restatement present in this image: transformers' Qwen3.5 torch fallbacks for the
    chunked and the recurrent gated delta rule (they scale q by 1/sqrt(Dk) internally; we undo that on input)."""
    mod = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    q, k, v, g, beta, s0 = _inputs(2, 150, 2, 64, seed=13)
    o, s = gdn.delta_rule_chunked(q, k, v, g, beta, 64, s0)
    qs = q * math.sqrt(64)
    o_tc, s_tc = mod.torch_chunk_gated_delta_rule(qs, k, v, g, beta, chunk_size=64, initial_state=s0,
                                                  output_final_state=True)
    o_tr, s_tr = mod.torch_recurrent_gated_delta_rule(qs, k, v, g, beta, initial_state=s0, output_final_state=True)
    # transformers computes in fp32 regardless of input dtype
    rel = lambda a, b: ((a.double() - b.double()).norm() / b.double().norm()).item()
    assert rel(o_tc, o) < 1e-5 and rel(s_tc, s) < 1e-5
    assert rel(o_tr, o) < 1e-5 and rel(s_tr, s) < 1e-5


def _gqa_inputs(B, T, G, R, D, seed):
    gen = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)
    q = mk(B, T, G, R, D)
    k = torch.nn.functional.normalize(mk(B, T, G, D), dim=-1)
    v = mk(B, T, G, D)
    g = -torch.rand(B, T, G, generator=gen, dtype=torch.float64) * 0.5
    beta = torch.rand(B, T, G, generator=gen, dtype=torch.float64)
    s0 = mk(B, G, D, D) * 0.3
    return q, k, v, g, beta, s0


def test_gqa_grads_gradcheck():
    """The oracle's backward (autograd of delta_rule_gqa) against finite differences of its forward, all six inputs,
    a sequence that is not a multiple of the chunk."""
    q, k, v, g, beta, s0 = (x.requires_grad_(True) for x in _gqa_inputs(1, 19, 2, 2, 4, seed=20))
    f = lambda *a: gdn.delta_rule_gqa(*a[:5], chunk=8, state=a[5])
    assert torch.autograd.gradcheck(f, (q, k, v, g, beta, s0), eps=1e-6, atol=1e-6)


def test_gqa_grads_match_token_recurrence():
    """delta_rule_gqa_grads equals autograd through the brute-force token recurrence on the R-repeated heads (the
    repeats' gradients summed), an independent formulation of the same function."""
    B, T, G, R, D = 2, 37, 2, 3, 8
    q, k, v, g, beta, s0 = _gqa_inputs(B, T, G, R, D, seed=21)
    gen = torch.Generator().manual_seed(22)
    do = torch.randn(B, T, G, R, D, generator=gen, dtype=torch.float64)
    ds = torch.randn(B, G, D, D, generator=gen, dtype=torch.float64)
    got = gdn.delta_rule_gqa_grads(q, k, v, g, beta, s0, do, ds, chunk=16)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v, g, beta, s0)]
    rep = lambda z: z.repeat_interleave(R, 2)
    o, s = gdn.delta_rule_recurrent(xs[0].reshape(B, T, G * R, D), rep(xs[1]), rep(xs[2]), rep(xs[3]), rep(xs[4]),
                                    xs[5].repeat_interleave(R, 1))
    # every repeat carries the same state; the final state of KV head g is that of its first query head
    loss = (o.reshape(B, T, G, R, D) * do).sum() + (s[:, ::R] * ds).sum()
    want = torch.autograd.grad(loss, xs)
    for a, b in zip(got, want):
        assert ((a - b).norm() / b.norm()).item() < 1e-10


def test_gqa_grads_chunk_invariant():
    B, T, G, R, D = 1, 50, 1, 2, 8
    q, k, v, g, beta, s0 = _gqa_inputs(B, T, G, R, D, seed=23)
    gen = torch.Generator().manual_seed(24)
    do = torch.randn(B, T, G, R, D, generator=gen, dtype=torch.float64)
    a = gdn.delta_rule_gqa_grads(q, k, v, g, beta, s0, do, None, chunk=8)
    b = gdn.delta_rule_gqa_grads(q, k, v, g, beta, s0, do, None, chunk=64)
    for x, y in zip(a, b):
        assert ((x - y).norm() / y.norm()).item() < 1e-10


def test_gqa_empty_sequence_keeps_state():
    """A sequence of no tokens: no output rows, the initial state unchanged."""
    q, k, v, g, beta, s0 = _gqa_inputs(1, 0, 2, 3, 8, seed=25)
    o, s = gdn.delta_rule_gqa(q, k, v, g, beta, 16, s0)
    assert o.shape == (1, 0, 2, 3, 8) and torch.equal(s, s0)
