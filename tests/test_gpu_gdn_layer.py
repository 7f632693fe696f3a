"""GPU parity of the native Gated DeltaNet layer (``heimdall_amd.gdn_layer``) against ``oracle.gdn_layer``:
the fused conv/norm/gate pass (``bf_gdn_conv_inputs``), ``bf_gated_norm``, the whole module forward with its conv and
state caches (prefill, split prefill, single-token steps), and the packed variable-length core.

Tolerances: relative L2 <= 1e-4 for fp32 runs; <= 2e-2 for bf16 runs against the fp32 oracle on the same
bf16-rounded inputs."""
import pytest
import torch

from oracle import gdn_layer as ol

pytestmark = pytest.mark.gpu

TOL32, TOL16 = 1e-4, 2e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def inputs(seed, N, hk, hv, d, K, dtype, num_seqs=1):
    g = torch.Generator().manual_seed(seed)
    C = (2 * hk + hv) * d
    return dict(z=torch.randn(N, C, generator=g).to(dtype), a=torch.randn(N, hv, generator=g) * 2,
                b=torch.randn(N, hv, generator=g), conv_w=torch.randn(C, K, generator=g) * 0.5,
                prefix=torch.randn(num_seqs, K - 1, C, generator=g).to(dtype),
                A_log=torch.randn(hv, generator=g) * 0.5 - 2, dt_bias=torch.randn(hv, generator=g))


@pytest.mark.parametrize("dtype,d", [(torch.float32, 64), (torch.bfloat16, 128), (torch.bfloat16, 256)])
def test_conv_inputs_packed_with_prefix(dev, dtype, d):
    from heimdall_amd.gdn_layer import conv_inputs
    hk, hv, K = 2, 4, 4
    lens = [5, 1, 70, 2]                        # sequences shorter than the conv, and one spanning many rows
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    N = int(cu[-1])
    c = inputs(1, N, hk, hv, d, K, dtype, num_seqs=len(lens))
    print(f"conv_inputs {dtype} d={d} lens={lens}", flush=True)
    got = conv_inputs(c["z"].to(dev), c["conv_w"].to(dev), c["prefix"].to(dev), c["a"].to(dev), c["b"].to(dev),
                      c["A_log"].to(dev), c["dt_bias"].to(dev), hk, hv, d, cu_seqlens=cu.to(dev),
                      out_dtype=torch.float32)
    tol = TOL32 if dtype == torch.float32 else TOL16
    for s in range(len(lens)):
        lo, hi = int(cu[s]), int(cu[s + 1])
        ref = ol.conv_inputs(c["z"][None, lo:hi].float(), c["conv_w"], c["prefix"][s:s + 1].float(),
                             c["a"][None, lo:hi], c["b"][None, lo:hi], c["A_log"], c["dt_bias"], hk, hv, d)
        for name, x, r in zip("qkvgb", got, ref):
            err = rel(x[lo:hi], r[0])
            assert err < tol, (s, name, err)


def test_conv_inputs_no_prefix_and_bf16_outputs(dev):
    from heimdall_amd.gdn_layer import conv_inputs
    hk, hv, d, K, N = 1, 3, 128, 4, 33
    c = inputs(2, N, hk, hv, d, K, torch.bfloat16)
    cu = torch.tensor([0, N], dtype=torch.int32, device=dev)
    q, k, v, g, beta = conv_inputs(c["z"].to(dev), c["conv_w"].to(dev), None, c["a"].to(dev), c["b"].to(dev),
                                   c["A_log"].to(dev), c["dt_bias"].to(dev), hk, hv, d, cu_seqlens=cu)
    assert q.dtype == torch.bfloat16
    ref = ol.conv_inputs(c["z"][None].float(), c["conv_w"], None, c["a"][None], c["b"][None], c["A_log"],
                         c["dt_bias"], hk, hv, d)
    for x, r in zip((q, k, v, g, beta), ref):
        assert rel(x, r[0]) < TOL16


@pytest.mark.parametrize("dtype,odt", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                       (torch.bfloat16, torch.bfloat16)])
def test_gated_norm(dev, dtype, odt):
    from heimdall_amd.gdn_layer import gated_norm
    g = torch.Generator().manual_seed(3)
    o = torch.randn(7, 5, 128, generator=g).to(odt)
    z = torch.randn(7, 5, 128, generator=g).to(dtype)
    w = torch.randn(128, generator=g).to(dtype).float()
    print(f"gated_norm io={dtype} o={odt}", flush=True)
    got = gated_norm(o.to(dev), z.to(dev), w.to(dev))
    assert got.dtype == dtype
    ref = ol.gated_norm(o.float(), z.float(), w, bf16_points=dtype == torch.bfloat16)
    assert rel(got, ref) < (TOL32 if dtype == torch.float32 else 5e-3)


def make_module(dev, dtype, d_model=96, hk=2, hv=4, d=64, seed=4):
    from heimdall_amd.gdn_layer import GatedDeltaNet, GdnLayerConfig
    torch.manual_seed(seed)
    m = GatedDeltaNet(GdnLayerConfig(d=d_model, lin_hk=hk, lin_hv=hv, lin_dk=d, lin_dv=d))
    with torch.no_grad():
        m.conv1d.weight.normal_(0, 0.5)
        m.A_log.normal_(-2, 0.5)
        m.dt_bias.normal_()
        m.norm.weight.normal_(1, 0.2)
    return m.to(device=dev, dtype=dtype)


def module_oracle(m, x, cache):
    """The module forward on the oracle: projections in fp32 from the module's (dtype-rounded) weights."""
    c = m.c
    xf = x.float().cpu()
    p = {n: t.detach().float().cpu() for n, t in m.named_parameters()}
    B, T, _ = x.shape
    z = xf @ p["in_proj_qkv.weight"].T
    a, b = xf @ p["in_proj_a.weight"].T, xf @ p["in_proj_b.weight"].T
    zg = xf @ p["in_proj_z.weight"].T
    o = ol.layer_core(z, a, b, zg, p["conv1d.weight"][:, 0], p["A_log"], p["dt_bias"], p["norm.weight"], c.lin_hk,
                      c.lin_hv, c.lin_dk, c.eps, cache=cache)
    return o @ p["out_proj.weight"].T


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_prefill_split_and_steps(dev, dtype):
    """Prefill of 150 tokens from an empty cache, then 70 more, then three single tokens, against the oracle with
    its own caches; every output and the final state."""
    m = make_module(dev, dtype)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 223, 96, generator=g).to(dtype)
    cache, ocache = {}, {}
    tol = TOL32 if dtype == torch.float32 else TOL16
    for lo, hi in ((0, 150), (150, 220), (220, 221), (221, 222), (222, 223)):
        print(f"module {dtype} tokens {lo}:{hi}", flush=True)
        y = m(x[:, lo:hi].to(dev), cache)
        y_ref = module_oracle(m, x[:, lo:hi], ocache)
        assert rel(y, y_ref) < tol, (lo, hi, rel(y, y_ref))
        assert rel(cache["S"], ocache["S"]) < tol
        assert rel(cache["conv"].float(), ocache["conv"].float()) < tol


def test_module_without_cache(dev):
    m = make_module(dev, torch.bfloat16, d_model=64, hk=1, hv=2, d=128)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 300, 64, generator=g).bfloat16()
    y = m(x.to(dev))
    assert rel(y, module_oracle(m, x, None)) < TOL16


def test_packed_core_matches_per_sequence(dev):
    """``gdn_layer_packed`` over 4 packed sequences (one shorter than a chunk) with carried prefixes and states
    equals the oracle layer core run per sequence."""
    from heimdall_amd.gdn_layer import gdn_layer_packed
    m = make_module(dev, torch.bfloat16, d_model=64, hk=2, hv=4, d=64)
    c = m.c
    lens = [130, 40, 257, 64]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    N = int(cu[-1])
    g = torch.Generator().manual_seed(7)
    C = (2 * c.lin_hk + c.lin_hv) * c.lin_dk
    z = torch.randn(N, C, generator=g).bfloat16()
    a, b = torch.randn(N, c.lin_hv, generator=g), torch.randn(N, c.lin_hv, generator=g)
    zg = torch.randn(N, c.lin_hv * c.lin_dv, generator=g).bfloat16()
    prefix = torch.randn(4, c.conv_k - 1, C, generator=g).bfloat16()
    s0 = torch.randn(4, c.lin_hv, c.lin_dk, c.lin_dv, generator=g) * 0.1
    out, s = gdn_layer_packed(m, z.to(dev), a.to(dev), b.to(dev), zg.to(dev), cu.to(dev), prefix.to(dev),
                              s0.to(dev))
    p = {n: t.detach().float().cpu() for n, t in m.named_parameters()}
    for i in range(4):
        lo, hi = int(cu[i]), int(cu[i + 1])
        cache = {"conv": prefix[i:i + 1].float(), "S": s0[i:i + 1]}
        ref = ol.layer_core(z[None, lo:hi].float(), a[None, lo:hi], b[None, lo:hi], zg[None, lo:hi].float(),
                            p["conv1d.weight"][:, 0], p["A_log"], p["dt_bias"], p["norm.weight"], c.lin_hk, c.lin_hv,
                            c.lin_dk, c.eps, cache=cache, bf16_points=True)
        assert rel(out[lo:hi], ref[0]) < TOL16, i
        assert rel(s[i], cache["S"][0]) < TOL16, i


@pytest.mark.parametrize("d,G,R", [(128, 4, 1), (64, 2, 2), (128, 1, 3)])
def test_fused_gated_norm_equals_two_passes(dev, d, G, R):
    """bf_gdn_fwd_gated (the GatedNorm applied by the output scan) against bf_gdn_fwd into o followed by
    bf_gated_norm: the same bits, over packed sequences of 70, 1, 200 and 129 tokens (a partial chunk, a one-token
    sequence) with an initial state, in single-segment and 2-chunk-segment scans; D = 256 and fp32 inputs are
    refused."""
    from heimdall_amd import _lib
    from heimdall_amd._device import gdn_forward
    from heimdall_amd.gdn_layer import gated_norm
    print(f"fused GatedNorm d={d} G={G} R={R}", flush=True)
    lens = [70, 1, 200, 129]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32, device=dev)
    N, H = sum(lens), G * R
    gen = torch.Generator(device=dev).manual_seed(3 + d + R)
    q = torch.randn(N, H, d, device=dev, generator=gen).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(N, G, d, device=dev, generator=gen), dim=-1).bfloat16()
    v = torch.randn(N, G, d, device=dev, generator=gen).bfloat16()
    g = -torch.rand(N, G, device=dev, generator=gen) * 0.1
    beta = torch.sigmoid(torch.randn(N, G, device=dev, generator=gen))
    s0 = torch.randn(4, G, d, d, device=dev, generator=gen) * 0.1
    zg = torch.randn(N, H, d, device=dev, generator=gen).bfloat16()
    w = torch.rand(d, device=dev, generator=gen) + 0.5
    for L in (0, 2):
        o, s = gdn_forward(q, k, v, g, beta, num_seqs=4, cu_seqlens=cu, initial_state=s0, scale=d ** -0.5,
                           out_dtype=torch.bfloat16, segment_chunks=L)
        ref = gated_norm(o, zg, w, 1e-6)
        out, sf = gdn_forward(q, k, v, g, beta, num_seqs=4, cu_seqlens=cu, initial_state=s0, scale=d ** -0.5,
                              segment_chunks=L, gated_norm=(zg, w, 1e-6))
        assert out.dtype == torch.bfloat16 and torch.isfinite(out.float()).all()
        assert torch.equal(out, ref), (L, (out.float() - ref.float()).abs().max().item())
        assert torch.equal(sf, s), L
    with pytest.raises(_lib.BifrostError):
        gdn_forward(q.float(), k.float(), v.float(), g, beta, num_seqs=4, cu_seqlens=cu, gated_norm=(zg, w, 1e-6))
    lib = _lib.load()
    assert lib.bf_gdn_fwd_gated(*([None] * 6), 1, 64, 1, 1, 256, 1.0, None, None, None, 1e-6, None, None, 0,
                                None, 0, _lib.PHASE_ALL, None) == -2          # BF_STATUS_UNSUPPORTED
