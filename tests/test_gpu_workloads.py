"""GPU parity at the full sizes of the benchmarked workloads, against the CPU oracle on the same inputs.

- Converted layer, fp32: B=1, T=4096, H=16, G=4, D=256, W=2048 + 4 sinks; decay half-lives {2048, 45255, 1e6} tokens
  on KV heads 0-2 and a non-decaying (archival) head 3; beta = sigmoid(N(0,1)), gamma = sigmoid(N(0,1)); zero
  initial state. One call from an empty cache, and the same tokens as two chunks through the cache.
- Packed native Gated DeltaNet: sequences {8192, 16384, 24576, 16384}, H=32, D=128, bf16, g ~ U[-5e-3, 0]: the
  delta rule alone and the layer core (conv, norms, gates, delta rule, gated norm), per sequence.
- Delta rule, B=1, T=32768, H=4, D=256, bf16 q/k/v (q unscaled, scale 1), g ~ U[-1e-3, 0]: whole sequence.
- Converted layer, bf16: B=1, T=32768, H=24, G=4, D=256, W=2048 + 4 sinks, against the oracle. At T=131072: the
  final state against the oracle's delta rule over the whole write stream, the last 2048 outputs against the
  oracle's student from the cache it holds at position T - 2048, and one call against two chunks through the cache.

Every full-size check records its error through the ``margin`` fixture: the session prints them all at the end.

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


def test_layer_fp32_T4096_H16_G4_D256(dev, margin):
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
    margin("o, one call", eo, TOL_F32)
    margin("S, one call", es, TOL_F32)
    compare_caches(c_ref, c_gpu, TOL_F32)
    c_ref, c_gpu = {}, {}
    with torch.no_grad():
        for a, e in ((0, 3000), (3000, T)):
            o_ref = olayer.student(m, *_split(args, a, e), a, c_ref)
            o = hibrit.student(mg, *(z.to(dev) for z in _split(args, a, e)), a, c_gpu)
            eo = rel(o, o_ref)
            say(f"  chunk {a}:{e} rel err o={eo:.2e}")
            margin(f"o, chunk {a}:{e}", eo, TOL_F32)
    margin("S, two chunks", rel(c_gpu["S"], c_ref["S"]), TOL_F32)
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


def test_varlen_delta_rule_packed_H32_D128_bf16(dev, margin):
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
        margin(f"o, sequence {i} ({e - a} tokens)", eo, TOL_BF16)
        margin(f"S, sequence {i}", es, TOL_BF16)


def test_gdn_layer_core_packed_H32_D128_bf16(dev, margin):
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
        margin(f"out, sequence {i} ({hi - lo} tokens)", eo, TOL_BF16)
        margin(f"S, sequence {i}", es, TOL_BF16)


def test_delta_rule_T32768_H4_D256_bf16_against_oracle(dev, margin):
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
    margin("o", eo, TOL_BF16)
    margin("o, last 2048 tokens", tail, TOL_BF16)
    margin("S", es, TOL_BF16)


def _layer_bf16_args(T, seed):
    H, G, D = 24, 4, 256
    return spectrum_inputs(1, T, H, G, D, seed, torch.bfloat16)


@pytest.mark.timeout(600)
def test_layer_bf16_T32768_H24_G4_D256_against_oracle(dev, margin):
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
    tail = rel(o[:, -2048:], o_ref[:, -2048:])
    say(f"  rel err o={eo:.2e} (last 2048 tokens {tail:.2e}) S={es:.2e} (oracle {time.time() - t0:.1f} s)")
    margin("o", eo, TOL_BF16)
    margin("o, last 2048 tokens", tail, TOL_BF16)
    margin("S", es, TOL_BF16)
    compare_caches(c_ref, c_gpu, TOL_BF16)


@pytest.mark.timeout(900)
def test_layer_bf16_T131072_H24_against_oracle(dev, margin):
    """T = 131072, the long-context workload (bf16, W = 2048 + 4 sinks, the decay spectrum), one call from an empty
    cache (about 128 composed scan segments in the memory branch), pinned to the oracle where it finishes in seconds:

    - the final state against the oracle's chunked delta rule (gdn.delta_rule_chunked, fp32) over the write stream
      the layer builds, km, v, g, beta of tokens 0 .. T - W - 1 (query W + i reads the state after writing token i),
      run in two pieces: tokens 0 .. T - 2048 - W - 1, giving S_mid, then the rest from S_mid;
    - the last 2048 outputs against the oracle's student (layer.student) called on that chunk at position T - 2048
      with the cache the layer holds there: S_mid, the ring of positions T - 4096 .. T - 2049 and the 4 sinks (the
      write stream's km, g, beta come from the oracle's own mem_inputs);
    - one call equals a 70000-token call followed by a 61072-token call through the cache (outputs, state, ring)."""
    import types
    from heimdall_amd import hibrit
    H, G, D, W, S, T = 24, 4, 256, 2048, 4, 131072
    say(f"layer bf16 B=1 T={T} H={H} G={G} D={D} W={W}+{S}: against the oracle at the end of the sequence")
    m = spectrum_core(H, G, D, W, S, (2048.0, 45255.0, 1e6, None))
    mg = _copy_core(m, dev)
    t0 = time.time()
    args = spectrum_inputs(1, T, H, G, D, 2, torch.bfloat16)
    argd = tuple(z.to(dev) for z in args)
    say(f"  inputs {time.time() - t0:.1f} s")
    c1 = {}
    with torch.no_grad():
        o = hibrit.student(mg, *argd, 0, c1)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    o_last, s_gpu = o[:, -2048:].cpu(), c1["S"].cpu()
    # the oracle's write stream: km, g, beta of tokens 0 .. T - W - 1 (a one-query-head view of the core keeps the
    # oracle's mem_inputs from projecting all 24 query heads, which the stream does not use)
    x, q, k, v, qr, kr = args
    m1 = types.SimpleNamespace(c=m.c, fq=m.fq[:1], fk=m.fk, ab=m.ab, A_log=m.A_log, dt_bias=m.dt_bias,
                               decay_mask=m.decay_mask, sinks=m.sinks)
    n = T - W
    parts = []
    with torch.no_grad():
        for a in range(0, n, 16384):
            e = min(a + 16384, n)
            _, km, g, beta = olayer.mem_inputs(m1, x[:, a:e], q[:, a:e, :1].float(), k[:, a:e].float(),
                                               torch.arange(a, e))
            parts.append((km, g, beta))
    km = torch.cat([p_[0] for p_ in parts], 1)
    g = torch.cat([p_[1] for p_ in parts], 1)
    beta = torch.cat([p_[2] for p_ in parts], 1)
    vv = v[:, :n].float()
    p0 = T - 2048
    n_mid = p0 - W
    say(f"  write stream {time.time() - t0:.1f} s")
    with torch.no_grad():
        _, s_mid = gdn.delta_rule_chunked(torch.zeros(1, n_mid, G, D), km[:, :n_mid], vv[:, :n_mid], g[:, :n_mid],
                                          beta[:, :n_mid], 64)
        _, s_fin = gdn.delta_rule_chunked(torch.zeros(1, n - n_mid, G, D), km[:, n_mid:], vv[:, n_mid:],
                                          g[:, n_mid:], beta[:, n_mid:], 64, initial_state=s_mid)
    es = rel(s_gpu, s_fin)
    say(f"  oracle delta rule over {n} writes {time.time() - t0:.1f} s: rel err S={es:.2e}")
    margin("S after 131072 tokens (oracle delta rule)", es, TOL_BF16)
    # the oracle's student on the last 2048 tokens from the cache at position T - 2048 (T - 4096 is a multiple of W,
    # so position p of the ring sits at slot p - (T - 4096))
    vt = v.transpose(1, 2)
    c_ref = dict(sink_k=kr[:, :, :S].float(), sink_v=vt[:, :, :S].float(),
                 ring_k=kr[:, :, p0 - W:p0].float().contiguous(), ring_v=vt[:, :, p0 - W:p0].float().contiguous(),
                 ring_km=km[:, p0 - W:p0].contiguous(), ring_g=g[:, p0 - W:p0].contiguous(),
                 ring_beta=beta[:, p0 - W:p0].contiguous(), ring_pos=torch.arange(p0 - W, p0), S=s_mid.clone())
    with torch.no_grad():
        o_ref = olayer.student(m, *(z.float() for z in _split(args, p0, T)), p0, c_ref)
    eo = rel(o_last, o_ref)
    say(f"  oracle student on the last 2048 tokens {time.time() - t0:.1f} s: rel err o={eo:.2e}")
    margin("o, last 2048 of 131072 tokens (oracle student from the cache)", eo, TOL_BF16)
    margin("S after 131072 tokens (oracle student's write)", rel(s_gpu, c_ref["S"]), TOL_BF16)
    del o_ref, c_ref, km, g, beta, vv
    # one call against two chunks through the cache
    c2 = {}
    with torch.no_grad():
        h = 70000
        oa = hibrit.student(mg, *_split(argd, 0, h), 0, c2)
        ob = hibrit.student(mg, *_split(argd, h, T), h, c2)
    torch.cuda.synchronize()
    e = rel(torch.cat((oa, ob), 1), o)
    es2 = rel(c2["S"], c1["S"])
    say(f"  one call vs 70000 + 61072: rel diff o={e:.2e} S={es2:.2e}")
    assert e < 5e-3 and es2 < 5e-3
    for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta"):
        assert rel(c2[key].float(), c1[key].float()) < 5e-3, key
    assert torch.equal(c2["ring_pos"], c1["ring_pos"])
