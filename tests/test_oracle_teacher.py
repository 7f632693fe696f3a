"""Pins for ``oracle.teacher`` (attention of the kept full-attention layers, with Quest-style retrieval).

The selection is checked against a per-query brute force written from the definition (candidates: the blocks that end
at or before p - W + 1; bound: the maximum over the KV head's query heads of sum_d max(q_d min_d, q_d max_d); the top
k of those), the way the reference's own ``test_retrieval_mask_reference`` checks it; the attention against the
library's ``scaled_dot_product_attention``."""
import pytest
import torch
import torch.nn.functional as F

from oracle import teacher as ot


def brute_force_mask(qr, kr, k, block, window, sinks):
    B, H, t, D = qr.shape
    G, n = kr.shape[1], kr.shape[2]
    R = H // G
    want = torch.zeros(B, H, t, n, dtype=torch.bool)
    for b in range(B):
        for g in range(G):
            for i in range(t):
                p = n - t + i
                blocks = [j for j in range((n - sinks) // block) if sinks + (j + 1) * block <= p - window + 1]
                ub = {}
                for j in blocks:
                    keys = kr[b, g, sinks + j * block:sinks + (j + 1) * block].double()
                    lo, hi = keys.min(0).values, keys.max(0).values
                    ub[j] = max(sum(max(float(qr[b, h, i, d]) * float(lo[d]), float(qr[b, h, i, d]) * float(hi[d]))
                                    for d in range(D)) for h in range(g * R, (g + 1) * R))
                top = sorted(blocks, key=lambda j: (-ub[j], j))[:k]
                row = torch.zeros(n, dtype=torch.bool)
                row[:sinks] = True
                row[sinks + len(blocks) * block:p + 1] = True
                for j in top:
                    row[sinks + j * block:sinks + (j + 1) * block] = True
                want[b, g * R:(g + 1) * R, i] = row
    return want


@pytest.mark.parametrize("B,H,G,D,n,t,k,block,window,sinks", [
    (1, 4, 2, 8, 50, 3, 2, 4, 6, 2),          # the reference test's geometry
    (2, 6, 3, 16, 90, 90, 3, 5, 9, 3),        # every position (queries inside the sinks too)
    (1, 8, 1, 8, 131, 7, 4, 8, 17, 0),        # no sinks, one KV head for 8 query heads
])
def test_retrieval_mask_matches_brute_force(B, H, G, D, n, t, k, block, window, sinks):
    g = torch.Generator().manual_seed(n)
    qr, kr = torch.randn(B, H, t, D, generator=g), torch.randn(B, G, n, D, generator=g)
    ret = dict(k=k, block=block, window=window, sinks=sinks)
    got = ot.retrieval_mask(qr, kr, ret)
    assert torch.equal(got, brute_force_mask(qr, kr, k, block, window, sinks))


def test_retrieval_all_blocks_is_causal():
    """k covering every block: each query at or past the sinks sees exactly the keys up to its position."""
    g = torch.Generator().manual_seed(1)
    B, H, G, D, n, t = 1, 4, 2, 16, 70, 30
    qr, kr = torch.randn(B, H, t, D, generator=g), torch.randn(B, G, n, D, generator=g)
    m = ot.retrieval_mask(qr, kr, dict(k=100, block=4, window=8, sinks=2))
    p = torch.arange(n - t, n)
    causal = torch.arange(n)[None, :] <= p[:, None]
    assert torch.equal(m, causal[None, None].expand_as(m))


def test_retrieval_k0_keeps_sinks_and_window():
    g = torch.Generator().manual_seed(2)
    B, H, G, D, n, t, S, W, L = 1, 2, 1, 8, 100, 5, 4, 10, 8
    qr, kr = torch.randn(B, H, t, D, generator=g), torch.randn(B, G, n, D, generator=g)
    m = ot.retrieval_mask(qr, kr, dict(k=0, block=L, window=W, sinks=S))
    for i in range(t):
        p = n - t + i
        nc = (p - W + 1 - S) // L
        row = torch.zeros(n, dtype=torch.bool)
        row[:S] = True
        row[S + nc * L:p + 1] = True
        assert torch.equal(m[0, 0, i], row)
        assert p + 1 - (S + nc * L) >= W             # the window holds W .. W + L - 1 keys
        assert p + 1 - (S + nc * L) <= W + L - 1


@pytest.mark.parametrize("t,n", [(40, 40), (1, 40), (6, 40)])
def test_teacher_matches_library_sdpa(t, n):
    g = torch.Generator().manual_seed(t)
    B, H, G, D = 2, 6, 2, 32
    qr = torch.randn(B, H, t, D, generator=g)
    kr = torch.randn(B, G, n, D, generator=g)
    v = torch.randn(B, n, G, D, generator=g)
    cache = {}
    if n > t:
        ot.teacher(torch.randn(B, H, n - t, D, generator=g), kr[:, :, :n - t], v[:, :n - t], cache)
    o = ot.teacher(qr, kr[:, :, n - t:], v[:, n - t:], cache)
    mask = torch.arange(n)[None, :] <= torch.arange(n - t, n)[:, None]
    k = kr.repeat_interleave(H // G, 1)
    vv = v.transpose(1, 2).repeat_interleave(H // G, 1)
    ref = F.scaled_dot_product_attention(qr.double(), k.double(), vv.double(), attn_mask=mask).transpose(1, 2)
    assert torch.allclose(o, ref, atol=1e-10)
    assert cache["k"].shape == (B, G, n, D)


def test_teacher_decode_steps_equal_one_causal_call():
    g = torch.Generator().manual_seed(3)
    B, H, G, D, n = 1, 4, 1, 16, 25
    qr, kr, v = torch.randn(B, H, n, D, generator=g), torch.randn(B, G, n, D, generator=g), \
        torch.randn(B, n, G, D, generator=g)
    whole = ot.teacher(qr, kr, v, None)
    cache = {}
    steps = [ot.teacher(qr[:, :, :10], kr[:, :, :10], v[:, :10], cache)]
    steps += [ot.teacher(qr[:, :, i:i + 1], kr[:, :, i:i + 1], v[:, i:i + 1], cache) for i in range(10, n)]
    assert torch.allclose(torch.cat(steps, 1), whole, atol=1e-12)
