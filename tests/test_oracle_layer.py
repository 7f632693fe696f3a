"""Pins the oracle's converted-layer student path: per-token brute force (write-on-exit, read, mix), chunked cache ==
full (``Heimdall/tests/test_hibrit.py:78-90``), memory off before the window fills (``:112-120``), constant cache
size (``:93-109``), the closed-form conversion init (``:217-228``) and, when present, golden vectors written by the
reference itself (``tests/golden/student_tiny.npz``)."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import layer

GOLDEN = Path(__file__).resolve().parent / "golden"


class Mod:
    pass


def make_module(h=4, hkv=2, dh=16, d=32, window=8, sinks=2, archival=1, seed=0, dtype=torch.float64,
                trained=True):
    """Converted-layer parameters; ``trained`` perturbs them away from the init like the reference's ``_converted``
    fixture (``Heimdall/tests/test_hibrit.py:50-59``)."""
    m = Mod()
    m.c = layer.Cfg(h, hkv, dh, d)
    gen = torch.Generator().manual_seed(seed)
    layer.convert_params(m, window, sinks, archival, gen, dtype)
    if trained:
        with torch.no_grad():
            for lin in (m.ab, m.mix):
                lin.weight.add_(torch.randn(lin.weight.shape, generator=gen, dtype=dtype) * 0.3)
                lin.bias.add_(torch.randn(lin.bias.shape, generator=gen, dtype=dtype) * 0.3)
            m.mix.bias.fill_(0.5)
            m.fq = m.fq + torch.randn(m.fq.shape, generator=gen, dtype=dtype) * 0.1
            m.fk = m.fk + torch.randn(m.fk.shape, generator=gen, dtype=dtype) * 0.1
            m.mix_lse = torch.randn(h, generator=gen, dtype=dtype) * 0.3
    return m


def make_inputs(m, b, t, seed=1, dtype=torch.float64):
    c = m.c
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(b, t, c.d, generator=gen, dtype=dtype)
    q = torch.randn(b, t, c.h, c.dh, generator=gen, dtype=dtype)
    k = torch.randn(b, t, c.hkv, c.dh, generator=gen, dtype=dtype)
    v = torch.randn(b, t, c.hkv, c.dh, generator=gen, dtype=dtype)
    # RoPE'd copies stand in as independent tensors (the core takes them as given)
    qr = (q + 0.1 * torch.randn(q.shape, generator=gen, dtype=dtype)).transpose(1, 2).contiguous()
    kr = (k + 0.1 * torch.randn(k.shape, generator=gen, dtype=dtype)).transpose(1, 2).contiguous()
    return x, q, k, v, qr, kr


def _split(args, a, e):
    x, q, k, v, qr, kr = args
    return x[:, a:e], q[:, a:e], k[:, a:e], v[:, a:e], qr[:, :, a:e], kr[:, :, a:e]


def test_student_equals_bruteforce():
    m = make_module()
    args = make_inputs(m, 2, 40)
    o = layer.student(m, *args, 0, None)
    o_bf = layer.student_bruteforce(m, *args)
    assert (o - o_bf).abs().max() < 1e-10


def test_student_gqa_r1_and_many_heads():
    m = make_module(h=6, hkv=2, dh=8, window=5, sinks=1)
    args = make_inputs(m, 1, 33, seed=4)
    assert (layer.student(m, *args, 0, None) - layer.student_bruteforce(m, *args)).abs().max() < 1e-10


@pytest.mark.parametrize("memory", [True, False])
def test_chunked_cache_equals_full(memory):
    m = make_module()
    args = make_inputs(m, 1, 61, seed=2)
    full = layer.student(m, *args, 0, None, memory)
    cache, outs, a = {}, [], 0
    for n in (5, 1, 13, 1, 1, 9, 30, 1):
        outs.append(layer.student(m, *_split(args, a, a + n), a, cache, memory))
        a += n
    assert (torch.cat(outs, 1) - full).abs().max() < 1e-10


def test_memory_branch_off_before_window():
    m = make_module()
    args = make_inputs(m, 1, 40, seed=3)
    s = layer.student(m, *args, 0, None, True)
    w = layer.student(m, *args, 0, None, False)
    assert (s[:, :8] - w[:, :8]).abs().max() < 1e-12
    assert (s[:, 8:] - w[:, 8:]).abs().max() > 1e-3


def test_cache_size_constant():
    m = make_module()
    args = make_inputs(m, 1, 160, seed=5)
    cache = {}
    layer.student(m, *_split(args, 0, 20), 0, cache)
    sizes = []
    for p in range(20, 160):
        layer.student(m, *_split(args, p, p + 1), p, cache)
        if p in (40, 159):
            sizes.append(sum(v.numel() * v.element_size() for v in cache.values() if torch.is_tensor(v)))
    assert sizes[0] == sizes[1]


def test_convert_init_closed_form():
    m = make_module(h=4, hkv=4, dh=16, window=16, archival=1, trained=False, dtype=torch.float32)
    life = math.log(2) / (m.A_log.exp() * torch.nn.functional.softplus(m.dt_bias))
    assert m.decay_mask[0] == 0 and torch.all(m.decay_mask[1:] == 1)
    assert torch.allclose(life, torch.logspace(math.log10(16), 6, 4), rtol=1e-3)
    assert torch.allclose(m.mem_scale, torch.full_like(m.mem_scale, 4.0))


@pytest.mark.skipif(not (GOLDEN / "student_tiny.npz").exists(), reason="golden fixture not generated")
def test_student_matches_reference_golden():
    """Golden vectors written by the reference's own ``HybridAttention._student`` (see tests/golden/)."""
    z = np.load(GOLDEN / "student_tiny.npz", allow_pickle=False)
    m = Mod()
    h, hkv, dh, d, w, s = (int(z[k]) for k in ("h", "hkv", "dh", "d", "window", "sinks"))
    m.c = layer.Cfg(h, hkv, dh, d)
    m.window, m.sinks = w, s
    t64 = lambda k: torch.from_numpy(z[k]).double()
    m.fq, m.fk, m.mix_lse, m.mem_scale = t64("fq"), t64("fk"), t64("mix_lse"), t64("mem_scale")
    m.A_log, m.dt_bias, m.decay_mask = t64("A_log"), t64("dt_bias"), t64("decay_mask")
    m.ab, m.mix = torch.nn.Linear(d, 2 * hkv).double(), torch.nn.Linear(d, h).double()
    with torch.no_grad():
        m.ab.weight.copy_(t64("ab_w")), m.ab.bias.copy_(t64("ab_b"))
        m.mix.weight.copy_(t64("mix_w")), m.mix.bias.copy_(t64("mix_b"))
    args = tuple(t64(k) for k in ("x", "q", "k", "v", "qr", "kr"))
    splits = [int(n) for n in z["splits"]]
    cache, outs, a = {}, [], 0
    for n in splits:
        outs.append(layer.student(m, *_split(args, a, a + n), a, cache))
        a += n
    o = torch.cat(outs, 1)
    ref = t64("o")
    assert (o - ref).abs().max() < 1e-4 * max(1.0, ref.abs().max().item())
    assert (cache["S"] - t64("S")).abs().max() < 1e-4
    full = layer.student(m, *args, 0, None)
    assert (full - t64("o_full")).abs().max() < 1e-4 * max(1.0, ref.abs().max().item())
