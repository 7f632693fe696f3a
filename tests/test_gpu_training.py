"""GPU parity of the conversion training's uses of the layer: stage A's differentiable student and the training
engine's loss on the kernels.

Mirrors the reference's test_motor_loss_and_grad_equal_stage_a (``Heimdall/tests/test_motor.py:42-65``): with every
position >= W weighted 1, the engine's segmented loss (``seq_loss``, ``motor.py:149-193``: the window precomputed once
without gradients by ``precompute``, ``:126-146``, the delta rule checkpointed per segment with the state carried)
equals stage A's ``rel_mse`` of ``distill_pair`` (``hibrit.py:434-439``, autograd through ``_student``), and so do the
gradients of the new parameters, for segments of several lengths. Here ``distill_pair`` runs
``heimdall_amd.hibrit.student`` under autograd (window kernel + ``motor.delta_rule_gqa`` with ``bf_gdn_bwd``), and the
engine's loss runs on ``heimdall_amd.motor.window_attention`` and ``heimdall_amd.motor.delta_rule_gqa``. Both are also
compared with autograd through the oracle's student in fp64 on the CPU.

The model around the layer is stood in for by fixed random tensors: the frozen projections' outputs (q, k, v, qr, kr,
the output gate) and the output projection W_o; the teacher's output yt is random.
Tolerances as the reference test: loss within 1e-5 relative, each gradient within 1e-4 of its largest entry.
"""
import math

import pytest
import torch
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from oracle import layer as olayer
from oracle import window as owin
from test_gpu_decode import make_core, make_inputs, rel

pytestmark = pytest.mark.gpu


def rel_mse(ys, yt, skip: int = 0):
    """``donustur_hibrit.rel_mse`` (``Heimdall/heimdall/donustur_hibrit.py:205-210``)."""
    if 0 < skip < ys.size(1):
        ys, yt = ys[:, skip:], yt[:, skip:]
    return (ys.float() - yt.float()).square().mean() / yt.float().square().mean().clamp(min=1e-8)


def params_of(m):
    return [m.fq, m.fk, m.ab.weight, m.ab.bias, m.mix.weight, m.mix.bias, m.mix_lse, m.mem_scale, m.A_log, m.dt_bias]


def setup(dev, H, G, D, d, W, S, T, seed):
    m = make_core(H, G, D, d, window=W, sinks=S, seed=seed)
    mg = make_core(H, G, D, d, window=W, sinks=S, seed=seed).to(dev)
    args = make_inputs(m, 1, T, seed=seed + 1)
    gen = torch.Generator().manual_seed(seed + 2)
    gate = torch.randn(1, T, H * D, generator=gen)
    W_o = torch.randn(d, H * D, generator=gen) / math.sqrt(H * D)
    yt = torch.randn(1, T, d, generator=gen)
    return m, mg, args, gate, W_o, yt


def stage_a_loss(student_fn, m, args, gate, W_o, yt):
    """distill_pair + rel_mse: the student's output after the gated output projection against the teacher's."""
    x, q, k, v, qr, kr = args
    B, T = x.shape[:2]
    o = student_fn(m, x, q, k, v, qr, kr, 0, None, True)
    ys = (o.reshape(B, T, -1) * torch.sigmoid(gate)) @ W_o.T
    return rel_mse(ys, yt, m.window)


def precompute(m, args, gate, W_o, yt, P, wq):
    """The record ``precompute`` (``motor.py:126-146``) keeps of one sequence, from the layer's inputs: the window
    output and LSE (``motor.window_attention``) at the loss positions P, the gate, the residual target."""
    from heimdall_amd import motor
    x, q, k, v, qr, kr = args
    with torch.no_grad():
        o_w, lse = motor.window_attention(m, qr, kr, v)
        owP = o_w[0, P].float()
        sg = torch.sigmoid(gate[0, P].float())
        base = (owP.reshape(len(P), -1) * sg) @ W_o.T
        yP = yt[0, P].float()
    return dict(kw=k[0], vw=v[0], xw=x[0], P=P, wq=wq.float(), qP=q[0, P], xP=x[0, P], owP=owP, sgP=sg,
                lseP=lse[0][:, P].T.float().contiguous(), rP=yP - base, den=(wq.float() * yP.square().sum(-1)).sum())


def seq_loss(a, d, seg: int, W_o):
    """The training engine's loss of one sequence (``motor.py:149-193``) with ``heimdall_amd.motor.delta_rule_gqa``:
    positions P in segments of ``seg`` tokens; at a segment boundary only the memory state is kept, and each segment is
    recomputed in the backward (checkpoint)."""
    from heimdall_amd.motor import delta_rule_gqa
    c = a.c
    G, R, D, W, S0 = c.hkv, c.h // c.hkv, c.dh, a.window, a.sinks
    T = d["kw"].size(0)
    P = d["P"]
    dev = W_o.device
    state = torch.zeros(1, G, D, D, device=dev)
    total = torch.zeros((), device=dev)

    def part(state, kw, vw, xw, n_zero, j0, sel, Pl):
        km = F.normalize(torch.einsum("tgd,gde->tge", kw.float(), a.fk), dim=-1)
        aa, bb = a.ab(xw.float()).chunk(2, dim=-1)
        gg = -a.A_log.exp() * F.softplus(aa + a.dt_bias) * a.decay_mask
        tok = torch.arange(j0, j0 + kw.size(0), device=dev)
        be = torch.sigmoid(bb) * (tok >= S0).float()[:, None]
        z = lambda u: F.pad(u, (0, 0) * (u.dim() - 1) + (n_zero, 0))
        wk, wv, wg, wb = z(km), z(vw.float()), z(gg), z(be)
        L = wk.size(0)
        qm = F.normalize(torch.einsum("phd,hde->phe", d["qP"][sel].float(), a.fq), dim=-1) * D ** -0.5
        qf = torch.zeros(L, G, R, D, device=dev).index_copy(0, Pl, qm.reshape(-1, G, R, D))
        o, state = delta_rule_gqa(qf[None], wk[None], wv[None], wg[None], wb[None], 64, state)
        om = o[0, Pl].reshape(-1, c.h, D)
        gam = torch.sigmoid(a.mix(d["xP"][sel].float()) + a.mix_lse * (d["lseP"][sel] - math.log(W)))
        delta = gam[..., None] * (a.mem_scale[:, None] * om - d["owP"][sel].float())
        y = (delta.reshape(len(Pl), -1) * d["sgP"][sel].float()) @ W_o.T
        return state, (d["wq"][sel] * (y - d["rP"][sel]).square().sum(-1)).sum()

    for t0 in range(0, T, seg):
        t1 = min(T, t0 + seg)
        if t1 <= W:
            continue
        sel = (P >= t0) & (P < t1)
        j0, j1 = max(0, t0 - W), t1 - W
        n_zero = (t1 - t0) - (j1 - j0)
        Pl = P[sel] - t0
        args = (state, d["kw"][j0:j1], d["vw"][j0:j1], d["xw"][j0:j1], n_zero, j0, sel, Pl)
        state, lp = checkpoint(part, *args, use_reentrant=False)
        total = total + lp
    return total / d["den"]


def _oracle_student(m, x, q, k, v, qr, kr, start, cache, memory):
    return olayer.student(m, x.double(), q.double(), k.double(), v.double(), qr.double(), kr.double(), start, cache,
                          memory)


def close_grads(got, ref, tol=1e-4):
    for i, (x, y) in enumerate(zip(got, ref)):
        x, y = x.detach().double().cpu(), y.detach().double().cpu()
        assert (x - y).abs().max() <= tol * max(1.0, y.abs().max().item()), (i, (x - y).abs().max().item())


@pytest.mark.parametrize("geom,segs", [((4, 2, 64, 32, 8, 2, 61), (16, 24, 128)),
                                       ((6, 2, 128, 48, 128, 4, 400), (100, 256))])
def test_engine_loss_and_grads_equal_stage_a(dev, geom, segs):
    from heimdall_amd import hibrit
    H, G, D, d, W, S, T = geom
    print(f"training H={H} G={G} D={D} W={W} S={S} T={T} segments {segs}", flush=True)
    m, mg, args, gate, W_o, yt = setup(dev, H, G, D, d, W, S, T, seed=3)
    ga = tuple(z.to(dev) for z in args)
    gate_g, W_o_g, yt_g = gate.to(dev), W_o.to(dev), yt.to(dev)
    for p in params_of(mg) + params_of(m):
        p.requires_grad_(True)
    # stage A on the GPU: autograd through the kernel student
    ref = stage_a_loss(hibrit.student, mg, ga, gate_g, W_o_g, yt_g)
    g_ref = torch.autograd.grad(ref, params_of(mg))
    # stage A on the oracle (fp64, CPU)
    ref_o = stage_a_loss(_oracle_student, m, args, gate.double(), W_o.double(), yt.double())
    g_or = torch.autograd.grad(ref_o, params_of(m))
    print(f"  stage A loss GPU {ref.item():.6f} oracle {ref_o.item():.6f}", flush=True)
    assert abs(ref.item() - ref_o.item()) < 1e-5 * max(1.0, ref_o.item())
    close_grads(g_ref, g_or)
    # the engine's loss over segments
    P = torch.arange(W, T, device=dev)
    rec = precompute(mg, ga, gate_g, W_o_g, yt_g, P, torch.ones(len(P), device=dev))
    for seg in segs:
        got = seq_loss(mg, rec, seg, W_o_g)
        g_got = torch.autograd.grad(got, params_of(mg))
        print(f"  seq_loss seg={seg}: {got.item():.6f}", flush=True)
        assert abs(got.item() - ref.item()) < 1e-5 * max(1.0, ref.item())
        close_grads(g_got, g_ref)


def test_student_autograd_chunks_match_oracle(dev):
    """The differentiable student through a cache (a prefill chunk past the window, a chunk reading the ring, single
    tokens): outputs equal the no-grad kernel path's, and the gradients of the new parameters of the summed chunk
    losses equal the oracle's."""
    from heimdall_amd import hibrit
    from test_gpu_decode import split
    print("training student autograd through a cache H=4 G=2 D=64 W=8 S=2 T=40", flush=True)
    m, mg, args, gate, W_o, yt = setup(dev, 4, 2, 64, 32, 8, 2, 40, seed=7)
    ga = tuple(z.to(dev) for z in args)
    for p in params_of(mg) + params_of(m):
        p.requires_grad_(True)
    c_g, c_o, c_n = {}, {}, {}
    loss_g = loss_o = 0.0
    a = 0
    for n in (20, 7, 1, 1, 11):
        og = hibrit.student(mg, *split(ga, a, a + n), a, c_g)
        oo = _oracle_student(m, *split(args, a, a + n), a, c_o, True)
        with torch.no_grad():
            on = hibrit.student(mg, *split(ga, a, a + n), a, c_n)
        assert rel(og, oo) < 1e-4 and rel(og, on) < 1e-5, (a, rel(og, oo), rel(og, on))
        sg = torch.sigmoid(gate[:, a:a + n].reshape(og.shape))
        loss_g = loss_g + (og * sg.to(dev)).square().sum()
        loss_o = loss_o + (oo * sg.double()).square().sum()
        a += n
    close_grads(torch.autograd.grad(loss_g, params_of(mg)), torch.autograd.grad(loss_o, params_of(m)))
    assert rel(c_g["S"], c_o["S"]) < 1e-4


def test_window_attention_and_window_binding(dev):
    """motor.window_attention (the cache-free window of precompute) and the ``_window`` binding with an explicit ring
    (positions before the chunk, some of them empty) against the oracle's window, fp32."""
    from heimdall_amd import hibrit, motor
    print("window_attention fp32 H=6 G=2 D=128 W=16 S=3 T=70 and _window over a ring", flush=True)
    m = make_core(6, 2, 128, 32, window=16, sinks=3)
    gen = torch.Generator().manual_seed(8)
    qr, kr = torch.randn(2, 6, 70, 128, generator=gen), torch.randn(2, 2, 70, 128, generator=gen)
    v = torch.randn(2, 70, 2, 128, generator=gen)
    o, lse = motor.window_attention(m, qr.to(dev), kr.to(dev), v.to(dev))
    o_ref, lse_ref = owin.window_attention_from_start(qr, kr, v.transpose(1, 2), 16, 3)
    assert rel(o, o_ref) < 1e-4 and (lse.cpu() - lse_ref).abs().max() < 1e-4
    # a chunk at position 37 after a ring of the previous W positions with two empty entries
    start, t = 37, 33
    pp = torch.arange(start - 16, start)
    ext_pos = torch.cat((pp, torch.arange(start, start + t)))
    ext_pos[3], ext_pos[9] = -1, -1
    ext_k, ext_v = torch.randn(2, 2, 16 + t, 128, generator=gen), torch.randn(2, 2, 16 + t, 128, generator=gen)
    q2 = torch.randn(2, 6, t, 128, generator=gen)
    sk, sv = torch.randn(2, 2, 3, 128, generator=gen), torch.randn(2, 2, 3, 128, generator=gen)
    pos = torch.arange(start, start + t)
    mg = make_core(6, 2, 128, 32, window=16, sinks=3).to(dev)
    o2, lse2 = hibrit.window(mg, q2.to(dev), ext_k.to(dev), ext_v.to(dev), ext_pos.to(dev), sk.to(dev), sv.to(dev),
                             pos.to(dev))
    o2_ref, lse2_ref = owin.window_attention_lse(q2, ext_k, ext_v, ext_pos, sk, sv, pos, 16, 3)
    assert rel(o2, o2_ref) < 1e-4 and (lse2.cpu() - lse2_ref).abs().max() < 1e-4


def test_window_inputs_requiring_grad_raise(dev):
    """The conversion's stage B (Heimdall/heimdall/donustur_hibrit.py:441-470) trains every converted layer end to end
    through HybridLM.hidden, so a layer's qr, kr and v require grad there; the window branch has no backward in this
    library, and the student refuses such inputs with BifrostError (it does not return a result whose window gradient
    would be missing). Stage A's case, the memory inputs and new parameters only, is differentiable (the tests above)."""
    from heimdall_amd import hibrit
    from heimdall_amd._device import BifrostError
    m = make_core(4, 2, 64, 32, window=8, sinks=2).to(dev)
    args = [z.to(dev) for z in make_inputs(m, 1, 20)]
    for i in (3, 4, 5):                                  # v, qr, kr
        a = [z.detach().clone() for z in args]
        a[i].requires_grad_(True)
        with pytest.raises(BifrostError, match="window branch has no backward"):
            hibrit.student(m, *a, 0, {})
