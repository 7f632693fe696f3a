"""GPU parity at the full sizes of the benchmarked workloads, against the CPU oracle on the same inputs.

- Converted layer, fp32: B=1, T=4096, H=16, G=4, D=256, W=2048 + 4 sinks; decay half-lives {2048, 45255, 1e6} tokens
  on KV heads 0-2 and a non-decaying (archival) head 3; beta = sigmoid(N(0,1)), gamma = sigmoid(N(0,1)); zero
  initial state. One call from an empty cache, and the same tokens as two chunks through the cache.
- Packed native Gated DeltaNet: sequences {8192, 16384, 24576, 16384}, H=32, D=128, bf16, g ~ U[-5e-3, 0]: the
  delta rule alone and the layer core (conv, norms, gates, delta rule, gated norm), per sequence.
- Delta rule, B=1, T=32768, H=4, D=256, bf16 q/k/v (q unscaled, scale 1), g ~ U[-1e-3, 0]: whole sequence.
- Converted layer, bf16: B=1, T=32768, H=24, G=4, D=256, W=2048 + 4 sinks, against the oracle; at T=131072 one call
  equals two chunks through the cache (the oracle would take minutes there).

Tolerances (relative L2 ||x - ref|| / ||ref|| on outputs and final states): <= 1e-4 for fp32 runs, <= 2e-2 for bf16
runs against the fp32 oracle evaluated on the same bf16-rounded inputs.
"""
import math
import time

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn, gdn_layer as ogl, layer as olayer

pytestmark = pytest.mark.gpu

TOL_F32, TOL_BF16 = 1e-4, 2e-2


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def say(msg):
    print(msg, flush=True)


def spectrum_core(H, G, D, W, S, lives, device="cpu"):
    """A converted core whose gates reproduce the workload's distributions exactly through the module's own
    parameters: d_model = G + H with x = [z_beta | z_gamma], beta = sigmoid(z_beta) (ab selects the first G columns of
    x, the decay logits a are 0), gamma = sigmoid(z_gamma) (mix selects the last H columns, mix_lse = 0), fq = fk = I,
    mem_scale = sqrt(D), and a constant log-decay g = -ln2 / life per KV head (decay_mask 0 on the archival heads,
    whose life is None)."""
    from heimdall_amd.hibrit import BifrostCore, CoreConfig
    m = BifrostCore(CoreConfig(H, G, D, G + H))
    m.convert(W, S, 0)
    with torch.no_grad():
        m.ab.weight.zero_()
        m.ab.bias.zero_()
        m.ab.weight[G:, :G] = torch.eye(G)
        m.mix.weight.zero_()
        m.mix.bias.zero_()
        m.mix.weight[:, G:] = torch.eye(H)
        sp = F.softplus(m.dt_bias)                       # g = -exp(A_log) softplus(0 + dt_bias) = -ln2 / life
        for h, life in enumerate(lives):
            if life is not None:
                m.A_log[h] = math.log(math.log(2.0) / life) - math.log(sp[h].item())
        m.decay_mask.copy_(torch.tensor([0.0 if life is None else 1.0 for life in lives]))
    return m.to(device)


def spectrum_inputs(B, T, H, G, D, seed, dtype):
    """q, k ~ N(0,1) L2-normalised per head, v ~ N(0,1), z_beta, z_gamma ~ N(0,1), drawn in that order; the window
    uses qr = q and kr = k (no rotary part)."""
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1)
    k = F.normalize(torch.randn(B, T, G, D, generator=gen), dim=-1)
    v = torch.randn(B, T, G, D, generator=gen)
    zb = torch.randn(B, T, G, generator=gen)
    zg = torch.randn(B, T, H, generator=gen)
    x = torch.cat((zb, zg), -1)
    q, k, v = (z.to(dtype) for z in (q, k, v))
    return x, q, k, v, q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()


def _split(args, a, e):
    x, q, k, v, qr, kr = args
    return x[:, a:e], q[:, a:e], k[:, a:e], v[:, a:e], qr[:, :, a:e], kr[:, :, a:e]


def _copy_core(m, dev):
    import copy
    mg = copy.deepcopy(m).to(dev)
    return mg


def test_layer_fp32_T4096_H16_G4_D256(dev):
    """fp32 converted layer at W=2048 + 4 sinks: one call from an empty cache, then the same tokens as chunks of 3000
    and 1096 through the cache (the second chunk reads the ring at production size); outputs and the final state
    within 1e-4 of the oracle, caches compared whole."""
    from heimdall_amd import hibrit
    from test_gpu_decode import compare_caches
    H, G, D, W, S, T = 16, 4, 256, 2048, 4, 4096
    say(f"layer fp32 B=1 T={T} H={H} G={G} D={D} W={W}+{S} spectrum (2048, 45255, 1e6, archival)")
    m = spectrum_core(H, G, D, W, S, (2048.0, 45255.0, 1e6, None))
    mg = _copy_core(m, dev)
    args = spectrum_inputs(1, T, H, G, D, 0, torch.float32)
    c_ref, c_gpu = {}, {}
    t0 = time.time()
    with torch.no_grad():
        o_ref = olayer.student(m, *args, 0, c_ref)
        say(f"  oracle full call {time.time() - t0:.1f} s")
        o = hibrit.student(mg, *(z.to(dev) for z in args), 0, c_gpu)
    eo, es = rel(o, o_ref), rel(c_gpu["S"], c_ref["S"])
    say(f"  full call rel err o={eo:.2e} S={es:.2e}")
    assert eo < TOL_F32 and es < TOL_F32
    compare_caches(c_ref, c_gpu, TOL_F32)
    c_ref, c_gpu = {}, {}
    with torch.no_grad():
        for a, e in ((0, 3000), (3000, T)):
            o_ref = olayer.student(m, *_split(args, a, e), a, c_ref)
            o = hibrit.student(mg, *(z.to(dev) for z in _split(args, a, e)), a, c_gpu)
            eo = rel(o, o_ref)
            say(f"  chunk {a}:{e} rel err o={eo:.2e}")
            assert eo < TOL_F32
    assert rel(c_gpu["S"], c_ref["S"]) < TOL_F32
    compare_caches(c_ref, c_gpu, TOL_F32)


PACKED = (8192, 16384, 24576, 16384)


def _packed_inputs(H, D, seed):
    N = sum(PACKED)
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(N, H, D, generator=gen).bfloat16()
    k = F.normalize(torch.randn(N, H, D, generator=gen), dim=-1).bfloat16()
    v = torch.randn(N, H, D, generator=gen).bfloat16()
    beta = torch.sigmoid(torch.randn(N, H, generator=gen))
    g = -torch.rand(N, H, generator=gen) * 5e-3
    return q, k, v, g, beta


def test_varlen_delta_rule_packed_H32_D128_bf16(dev):
    """kernels.delta_rule_varlen on four packed sequences {8192, 16384, 24576, 16384} (zero initial states) against the
    oracle run per sequence (the reference has no packed form: one call per sequence)."""
    from heimdall_amd import kernels
    H, D = 32, 128
    say(f"varlen delta rule bf16 lens={PACKED} H={H} D={D}")
    q, k, v, g, beta = _packed_inputs(H, D, 4)
    cu = [0]
    for n in PACKED:
        cu.append(cu[-1] + n)
    with torch.no_grad():
        o, s = kernels.delta_rule_varlen(*(z.to(dev)[None] for z in (q, k, v, g, beta)),
                                         torch.tensor(cu, dtype=torch.int32, device=dev))
    o = o[0].cpu()
    s = s.cpu()
    for i, (a, e) in enumerate(zip(cu[:-1], cu[1:])):
        t0 = time.time()
        o_ref, s_ref = gdn.delta_rule_chunked(*(z[a:e][None].float() for z in (q, k, v, g, beta)), 64)
        eo, es = rel(o[a:e], o_ref[0]), rel(s[i], s_ref[0])
        say(f"  sequence {i} ({e - a} tokens): rel err o={eo:.2e} S={es:.2e} (oracle {time.time() - t0:.1f} s)")
        assert eo < TOL_BF16 and es < TOL_BF16


def test_gdn_layer_core_packed_H32_D128_bf16(dev):
    """gdn_layer_packed (conv + SiLU + l2norm + gates, delta rule, gated norm) on the same four packed sequences,
    H = 32 key and value heads, D = 128, conv width 4, bf16, against the oracle layer core per sequence with the
    reference's bf16 rounding points."""
    from heimdall_amd.gdn_layer import GatedDeltaNet, GdnLayerConfig, gdn_layer_packed
    H, D, K = 32, 128, 4
    say(f"gdn layer core bf16 lens={PACKED} H={H} D={D} conv {K}")
    torch.manual_seed(5)
    m = GatedDeltaNet(GdnLayerConfig(d=64, lin_hk=H, lin_hv=H, lin_dk=D, lin_dv=D, conv_k=K))
    with torch.no_grad():
        m.conv1d.weight.normal_(0, 0.5)
        m.A_log.uniform_(-6, -2)
        m.dt_bias.normal_()
    m = m.to(dev).bfloat16()
    N = sum(PACKED)
    C = 3 * H * D
    gen = torch.Generator().manual_seed(6)
    z = torch.randn(N, C, generator=gen).bfloat16()
    a, b = torch.randn(N, H, generator=gen), torch.randn(N, H, generator=gen)
    zg = torch.randn(N, H * D, generator=gen).bfloat16()
    cu = torch.tensor([0] + list(torch.tensor(PACKED).cumsum(0)), dtype=torch.int32)
    with torch.no_grad():
        out, s = gdn_layer_packed(m, z.to(dev), a.to(dev), b.to(dev), zg.to(dev), cu.to(dev))
    out, s = out.cpu(), s.cpu()
    p = {n: t.detach().float().cpu() for n, t in m.named_parameters()}
    for i in range(len(PACKED)):
        lo, hi = int(cu[i]), int(cu[i + 1])
        cache = {}
        ref = ogl.layer_core(z[None, lo:hi].float(), a[None, lo:hi], b[None, lo:hi], zg[None, lo:hi].float(),
                             p["conv1d.weight"][:, 0], p["A_log"], p["dt_bias"], p["norm.weight"], H, H, D,
                             m.c.eps, cache=cache, bf16_points=True)
        eo, es = rel(out[lo:hi], ref[0]), rel(s[i], cache["S"][0])
        say(f"  sequence {i} ({hi - lo} tokens): rel err out={eo:.2e} S={es:.2e}")
        assert eo < TOL_BF16 and es < TOL_BF16


def test_delta_rule_T32768_H4_D256_bf16_against_oracle(dev):
    """The whole 32768-token sequence (31 scan segments composed on the GPU) against the oracle's sequential chunked
    form: the error of the segment composition does not grow past the bf16 bound over the full length."""
    from heimdall_amd import kernels
    B, T, H, D = 1, 32768, 4, 256
    say(f"delta rule bf16 B={B} T={T} H={H} D={D} q unscaled, g ~ U[-1e-3, 0]")
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(B, T, H, D, generator=gen).bfloat16()
    k = F.normalize(torch.randn(B, T, H, D, generator=gen), dim=-1).bfloat16()
    v = torch.randn(B, T, H, D, generator=gen).bfloat16()
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    g = -torch.rand(B, T, H, generator=gen) * 1e-3
    with torch.no_grad():
        o, s = kernels.delta_rule(*(z.to(dev) for z in (q, k, v, g, beta)))
    t0 = time.time()
    o_ref, s_ref = gdn.delta_rule_chunked(*(z.float() for z in (q, k, v, g, beta)), 64)
    o = o.cpu()
    eo, es = rel(o, o_ref), rel(s, s_ref)
    tail = rel(o[:, -2048:], o_ref[:, -2048:])
    say(f"  rel err o={eo:.2e} (last 2048 tokens {tail:.2e}) S={es:.2e} (oracle {time.time() - t0:.1f} s)")
    assert eo < TOL_BF16 and es < TOL_BF16 and tail < TOL_BF16


def _layer_bf16_args(T, seed):
    H, G, D = 24, 4, 256
    return spectrum_inputs(1, T, H, G, D, seed, torch.bfloat16)


@pytest.mark.timeout(600)
def test_layer_bf16_T32768_H24_G4_D256_against_oracle(dev):
    """The converted layer at the 32K prefill workload (bf16 activations, fp32 state, W = 2048 + 4 sinks, decay
    spectrum of the fp32 workload with G = 4) from an empty cache, against the oracle on the same bf16 values:
    outputs, the final state and the ring."""
    from heimdall_amd import hibrit
    from test_gpu_decode import compare_caches
    H, G, D, W, S, T = 24, 4, 256, 2048, 4, 32768
    say(f"layer bf16 B=1 T={T} H={H} G={G} D={D} W={W}+{S}")
    m = spectrum_core(H, G, D, W, S, (2048.0, 45255.0, 1e6, None))
    mg = _copy_core(m, dev)
    args = _layer_bf16_args(T, 1)
    c_gpu = {}
    with torch.no_grad():
        o = hibrit.student(mg, *(z.to(dev) for z in args), 0, c_gpu).cpu()
    c_ref = {}
    t0 = time.time()
    with torch.no_grad():
        o_ref = olayer.student(m, *(z.float() for z in args), 0, c_ref)
    eo, es = rel(o, o_ref), rel(c_gpu["S"], c_ref["S"])
    say(f"  rel err o={eo:.2e} S={es:.2e} (oracle {time.time() - t0:.1f} s)")
    assert eo < TOL_BF16 and es < TOL_BF16
    compare_caches(c_ref, c_gpu, TOL_BF16)


def test_layer_bf16_T131072_H24_one_call_equals_two_chunks(dev):
    """T = 131072 (the long-context workload): one call from an empty cache equals a 70000-token call followed by a
    61072-token call through the cache (outputs, state and ring), the memory branch active throughout; outputs finite."""
    from heimdall_amd import hibrit
    H, G, D, W, S, T = 24, 4, 256, 2048, 4, 131072
    say(f"layer bf16 B=1 T={T} H={H} G={G} D={D} W={W}+{S}: one call vs two chunks")
    m = spectrum_core(H, G, D, W, S, (2048.0, 45255.0, 1e6, None), device=dev)
    gen = torch.Generator(device=dev).manual_seed(2)
    q = F.normalize(torch.randn(1, T, H, D, device=dev, generator=gen), dim=-1).bfloat16()
    k = F.normalize(torch.randn(1, T, G, D, device=dev, generator=gen), dim=-1).bfloat16()
    v = torch.randn(1, T, G, D, device=dev, generator=gen).bfloat16()
    x = torch.randn(1, T, G + H, device=dev, generator=gen)
    qr, kr = q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
    args = (x, q, k, v, qr, kr)
    c1, c2 = {}, {}
    with torch.no_grad():
        o = hibrit.student(m, *args, 0, c1)
        h = 70000
        oa = hibrit.student(m, *_split(args, 0, h), 0, c2)
        ob = hibrit.student(m, *_split(args, h, T), h, c2)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    e = rel(torch.cat((oa, ob), 1), o)
    es = rel(c2["S"], c1["S"])
    say(f"  rel diff o={e:.2e} S={es:.2e}")
    assert e < 5e-3 and es < 5e-3
    for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta"):
        assert rel(c2[key].float(), c1[key].float()) < 5e-3, key
    assert torch.equal(c2["ring_pos"], c1["ring_pos"])
