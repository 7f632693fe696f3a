"""Pins for ``oracle.formats``: the llama.cpp state row of a converted layer and the GGUF tensors of a conversion.

The row is checked against the sizes the patch states for the production geometry, against ggml's mul_mat
convention for the delta block (the layer reads o_mem = mul_mat(state, qm)), against the slot rule slot = S + pos
mod (W + 1) and the ggml views of the K / V planes written as explicit index arithmetic, and by a round trip. The
GGUF tensors are checked by using them the way llama.cpp's graph does and comparing with the reference's memory
inputs."""
import types

import numpy as np
import torch
import torch.nn.functional as F

from oracle import formats as of
from oracle import layer as ol


def test_state_size_production_geometry():
    # G = 4, D = 256, W = 2048, S = 4: LR = ceil(2054 / 32) * 32 = 2080 slots, C = 3 * 1024 + 8 = 3080 channels,
    # LR * (C + 2 G D) + D^2 G = 2080 * 5128 + 262144 floats (43.7 MB per sequence per layer)
    assert of.region_slots(2048, 4) == 2080
    assert of.ring_channels(4, 256) == 3080
    assert of.state_floats(4, 256, 2048, 4) == 10_928_384


def random_cache(B, G, D, W, S, n, seed):
    g = torch.Generator().manual_seed(seed)
    c = dict(ring_k=torch.randn(B, G, W, D, generator=g), ring_v=torch.randn(B, G, W, D, generator=g),
             ring_km=torch.randn(B, W, G, D, generator=g), ring_g=-torch.rand(B, W, G, generator=g),
             ring_beta=torch.rand(B, W, G, generator=g), ring_pos=torch.full((W,), -1, dtype=torch.long),
             S=torch.randn(B, G, D, D, generator=g))
    for p in range(max(0, n - W), n):
        c["ring_pos"][p % W] = p
    ns = min(S, n)
    c["sink_k"], c["sink_v"] = torch.randn(B, G, ns, D, generator=g), torch.randn(B, G, ns, D, generator=g)
    return c


def test_delta_block_follows_ggml_mul_mat():
    """o_mem = ggml_mul_mat(state [D, D, G], qm [D, R, G]) contracts the state's first (fastest) axis with qm:
    read back that way, the block gives the reference's o = q S for every KV head."""
    B, G, D, W, S, n = 1, 2, 8, 6, 2, 9
    c = random_cache(B, G, D, W, S, n, seed=1)
    row = of.llama_state_row(c, 0, n, W, S)
    LR, C = of.region_slots(W, S), of.ring_channels(G, D)
    flat = row[LR * C + 2 * LR * G * D:]
    q = np.random.default_rng(2).standard_normal((G, D)).astype(np.float32)
    for g in range(G):
        # ggml: element (i0, i1, i2) of a [D, D, G] tensor at i0 + D (i1 + D i2); result[i1] = sum_i0 a[i0, i1] b[i0]
        o = np.array([sum(flat[i0 + D * (i1 + D * g)] * q[g, i0] for i0 in range(D)) for i1 in range(D)])
        assert np.allclose(o, q[g] @ c["S"][0, g].numpy(), atol=1e-5)


def test_slot_rule_and_plane_views():
    B, G, D, W, S = 1, 2, 4, 5, 2
    for n in (1, 3, 7, 13):                       # before and after the window fills, sinks partly present
        c = random_cache(B, G, D, W, S, n, seed=n)
        row = of.llama_state_row(c, 0, n, W, S)
        LR, C, GD = of.region_slots(W, S), of.ring_channels(G, D), G * D
        region = row[:LR * C].reshape(LR, C)
        for p in range(max(0, n - W), n):          # window rows at slot S + p mod (W + 1)
            r = region[S + p % (W + 1)]
            s = p % W
            assert np.array_equal(r[:GD], c["ring_k"][0, :, s].reshape(-1).numpy())
            assert np.array_equal(r[GD:2 * GD], c["ring_v"][0, :, s].reshape(-1).numpy())
            assert np.array_equal(r[2 * GD:3 * GD], c["ring_km"][0, s].reshape(-1).numpy())
            assert np.array_equal(r[3 * GD:], np.concatenate((c["ring_g"][0, s].numpy(), c["ring_beta"][0, s].numpy())))
        for j in range(min(S, n)):                  # sinks at slots 0 .. S - 1
            assert np.array_equal(region[j, :GD], c["sink_k"][0, :, j].reshape(-1).numpy())
        kp = row[LR * C:LR * C + LR * GD]          # ggml [D, LR, G]: (d, l, g) at d + D (l + LR g)
        vp = row[LR * C + LR * GD:LR * C + 2 * LR * GD]   # ggml [LR, D, G]: (l, d, g) at l + LR (d + D g)
        for g in range(G):
            for l in range(LR):
                for d in range(D):
                    assert kp[d + D * (l + LR * g)] == region[l, g * D + d]
                    assert vp[l + LR * (d + D * g)] == region[l, GD + g * D + d]


def test_row_roundtrip():
    B, G, D, W, S, n = 2, 2, 8, 7, 3, 20
    c = random_cache(B, G, D, W, S, n, seed=3)
    rows = np.stack([of.llama_state_row(c, b, n, W, S) for b in range(B)])
    back = of.cache_from_llama_rows(rows, n, W, S, G, D)
    for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta", "ring_pos", "sink_k", "sink_v", "S"):
        assert np.array_equal(back[key], c[key].numpy()), key


def test_gguf_tensors_reproduce_memory_inputs():
    """Used as llama.cpp's graph uses them (bifrost.patch: qm = mul_mat(fq, q) per head, g = softplus(a_in + dt) *
    a, beta = sigmoid(b_in)), the GGUF tensors give the reference's memory inputs (hibrit.py:327-334)."""
    torch.manual_seed(4)
    G, R, D, d = 2, 2, 8, 12
    m = types.SimpleNamespace(c=ol.Cfg(G * R, G, D, d))
    ol.convert_params(m, window=16, sinks=2, archival=1)
    with torch.no_grad():
        m.fq = torch.randn(G * R, D, D)
        m.fk = torch.randn(G, D, D)
        m.ab.weight.normal_()
        m.ab.bias.normal_()
    params = {"fq": m.fq, "fk": m.fk, "ab.weight": m.ab.weight, "ab.bias": m.ab.bias, "mix.weight": m.mix.weight,
              "mix.bias": m.mix.bias, "mix_lse": m.mix_lse, "mem_scale": m.mem_scale, "A_log": m.A_log,
              "dt_bias": m.dt_bias}
    t = of.gguf_tensors(params, archival=1)
    x, q, k = torch.randn(1, 5, d), torch.randn(1, 5, G * R, D), torch.randn(1, 5, G, D)
    pos = torch.arange(5)
    qm, km, g, beta = ol.mem_inputs(m, x, q, k, pos)
    # ggml_mul_mat(w [D_in, D_out] per head, z): out[e] = sum_i w[i + D e] z[i], w stored as the transposed fq
    qm_ggml = torch.einsum("hed,bthd->bthe", t["bifrost_fq"], q)
    assert torch.allclose(F.normalize(qm_ggml, dim=-1) * D ** -0.5, qm, atol=1e-5)
    km_ggml = torch.einsum("hed,bthd->bthe", t["bifrost_fk"], k)
    assert torch.allclose(F.normalize(km_ggml, dim=-1), km, atol=1e-5)
    ab = x @ t["bifrost_ab"].T + t["bifrost_ab_b"]
    g_ggml = F.softplus(ab[..., :G] + t["bifrost_dt"]) * t["bifrost_a"]
    assert torch.allclose(g_ggml, g, atol=1e-6)
    assert torch.equal(t["bifrost_a"][:1], torch.zeros(1))          # the archival head never decays
    beta_ggml = torch.sigmoid(ab[..., G:]) * (pos >= 2).float()[None, :, None]
    assert torch.allclose(beta_ggml, beta, atol=1e-6)
