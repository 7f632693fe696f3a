"""Drop-in GPU student path of the converted (Bifrost) attention layer.

Mirrors ``HybridAttention`` of the reference (``Heimdall/heimdall/hibrit.py:193-424``) for the part this package
accelerates: the same new-parameter names and conversion init (``convert``, ``hibrit.py:211-240``), the same
``_mem_inputs`` (``:327-334``) and a ``_student(x, q, k, v, qr, kr, start, cache, memory)`` with the reference's
signature and cache contract (keys ``sink_k, sink_v, ring_k, ring_v, ring_km, ring_g, ring_beta, ring_pos, S`` with
the same shapes and meaning, mutated in place), so a cache can move between the reference and this implementation.

The window + sink attention, the delta-rule memory and the gamma mix run in ``libbifrost_hip.so``:
  t == 1  -> ``bf_decode_fwd`` (one bandwidth-bound pass: state update, window read, mix, ring write)
  t > 1   -> ``bf_gdn_fwd`` (memory branch) then ``bf_window_fwd`` (window + sinks + LSE, fused gamma mix)
The frozen projections and the small per-token gate GEMMs (fq/fk, ab, mix) stay in PyTorch.

``student`` can be bound onto the reference class as a drop-in: ``HybridAttention._student = student``; likewise the
teacher path of the kept full-attention layers, ``HybridAttention._teacher = teacher`` and ``set_retrieval``
(``heimdall_amd.teacher``: KV-cache attention with Quest-style retrieval).
"""
import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from ._device import (BifrostError, check, compute_dtype, dtype_code, require_device, require_no_grad, stream_ptr,
                      workspace)
from .teacher import set_retrieval, teacher

NEW = ("fq", "fk", "ab", "mix", "mix_lse", "mem_scale", "A_log", "dt_bias")


class CoreConfig:
    """Head geometry with the reference's attribute names (``HybridConfig.h / hkv / dh / d``)."""

    def __init__(self, h: int, hkv: int, dh: int, d: int):
        if h % hkv:
            raise ValueError("query heads must be a multiple of KV heads")
        self.h, self.hkv, self.dh, self.d = h, hkv, dh, d


def n_archival(frac: float, hkv: int, mem_init: str = "long") -> int:
    """Never-forgetting memory heads (``hibrit.py:187-190``)."""
    n = int(frac * hkv)
    return max(1, n) if mem_init == "long" and frac > 0 else n


def _heads_matmul(x: torch.Tensor, f: torch.Tensor) -> torch.Tensor:
    """x [B, t, h, D] fp32, f [h, D, D] -> x_h f_h per head (a batched GEMM with contiguous operands)."""
    b, t, h, d = x.shape
    y = torch.matmul(x.permute(2, 0, 1, 3).reshape(h, b * t, d).contiguous(), f.float().contiguous())
    return y.reshape(h, b, t, d).permute(1, 2, 0, 3)


def mem_inputs(self, x, q, k, pos):
    """qm = normalize(q_h F_q,h) / sqrt(D); km = normalize(k_g F_k,g); g = -exp(A_log) softplus(a + dt_bias) mask;
    beta = sigmoid(b) [pos >= sinks]  (``hibrit.py:327-334``), all fp32."""
    dh = self.c.dh
    qm = F.normalize(_heads_matmul(q.float(), self.fq), dim=-1) * dh ** -0.5
    km = F.normalize(_heads_matmul(k.float(), self.fk), dim=-1)
    a, bb = F.linear(x.float(), self.ab.weight.float(), self.ab.bias.float()).chunk(2, dim=-1)
    g = -self.A_log.float().exp() * F.softplus(a + self.dt_bias.float()) * self.decay_mask.float()
    beta = torch.sigmoid(bb) * (pos >= self.sinks).float()[None, :, None]
    return qm, km, g, beta


def _f32(p: torch.Tensor) -> torch.Tensor:
    """A parameter as a contiguous fp32 tensor (itself when it already is one: no copy, read where it lies)."""
    p = p.detach()
    return p if p.dtype == torch.float32 and p.is_contiguous() else p.float().contiguous()


def _project_bf16(x: torch.Tensor, f: torch.Tensor, scale: float, out_dtype=torch.bfloat16) -> torch.Tensor:
    """bf16 x [B, t, nh, D] -> scale * normalize(x_h f_h) [B, t, nh, D] in out_dtype on bf_mem_project, which reads
    the projection f [nh, D, D] as the module holds it (fp32) on every call: nothing is cached between calls, so
    parameter writes of any kind (an optimizer step, ``p.data.copy_`` as the reference's apply_conversion makes,
    hibrit.py:798) reach the next call."""
    b, t, nh, d = x.shape
    if x.stride(-1) != 1 or (b > 1 and x.stride(0) != t * x.stride(1)):
        x = x.contiguous()
    out = torch.empty(b, t, nh, d, dtype=out_dtype, device=x.device)
    f = _f32(f)
    check(_lib.load().bf_mem_project(x.data_ptr(), b * t, nh, d, x.stride(1), x.stride(2), f.data_ptr(), float(scale),
                                     out.data_ptr(), _lib.DTYPE_BF16, dtype_code(out_dtype), stream_ptr(x.device)),
          "bf_mem_project")
    return out


def _gate_logits(self, x):
    """The two gate projections of a chunk, fp32: ab = ab(x) [B, t, 2G] (``hibrit.py:330``) and z = mix(x) [B, t, H]
    (the gamma logit, ``:409``). bf16 x with a row length that is a multiple of 8: one bf_gate_project pass over x (x
    exact, the weights as bf16 high + low parts, fp32 accumulation); otherwise fp32 PyTorch products."""
    G, H = self.c.hkv, self.c.h
    b, t, d = x.shape
    f32 = lambda p: p if p.dtype == torch.float32 and p.is_contiguous() else p.float().contiguous()
    if (x.dtype == torch.bfloat16 and d % 8 == 0 and x.stride(-1) == 1 and x.stride(1) % 8 == 0
            and (b == 1 or x.stride(0) == t * x.stride(1)) and x.data_ptr() % 16 == 0):
        ab = torch.empty(b, t, 2 * G, dtype=torch.float32, device=x.device)
        z = torch.empty(b, t, H, dtype=torch.float32, device=x.device)
        w0, b0 = f32(self.ab.weight.detach()), f32(self.ab.bias.detach())
        w1, b1 = f32(self.mix.weight.detach()), f32(self.mix.bias.detach())
        lib = _lib.load()
        nb = _lib.ctypes.c_size_t(0)
        check(lib.bf_gate_project_workspace_size(b * t, d, 2 * G + H, _lib.ctypes.byref(nb)),
              "bf_gate_project_workspace_size")
        ws = workspace(nb.value, x.device) if nb.value else None
        check(lib.bf_gate_project(x.data_ptr(), b * t, d, x.stride(1), w0.data_ptr(), b0.data_ptr(), 2 * G,
                                  ab.data_ptr(), w1.data_ptr(), b1.data_ptr(), H, z.data_ptr(),
                                  None if ws is None else ws.data_ptr(), nb.value, stream_ptr(x.device)),
              "bf_gate_project")
        return ab, z
    xf = x.float()
    ab = F.linear(xf, self.ab.weight.float(), self.ab.bias.float()).contiguous()
    z = F.linear(xf, self.mix.weight.float(), self.mix.bias.float()).contiguous()
    return ab, z


def _mem_inputs_bf16(self, ab, q, k, start: int, out_dtype=torch.bfloat16):
    """mem_inputs for bf16 activations (no autograd): qm, km from the fused projection kernel (out_dtype out, fp32
    accumulation and norm), the gates g, beta in fp32 from the ab projection ``ab`` [B, t, 2G] by bf_mem_gates
    (``hibrit.py:327-334``)."""
    dh, G = self.c.dh, self.c.hkv
    qm = _project_bf16(q, self.fq, dh ** -0.5, out_dtype)
    km = _project_bf16(k, self.fk, 1.0, out_dtype)
    b, t = ab.shape[:2]
    g = torch.empty(b, t, G, dtype=torch.float32, device=ab.device)
    beta = torch.empty_like(g)
    f32 = lambda p: p if p.dtype == torch.float32 and p.is_contiguous() else p.float().contiguous()
    A_log, dt_bias, mask = f32(self.A_log.detach()), f32(self.dt_bias.detach()), f32(self.decay_mask)
    check(_lib.load().bf_mem_gates(ab.data_ptr(), b * t, t, G, 2 * G, A_log.data_ptr(), dt_bias.data_ptr(),
                                   mask.data_ptr(), start, self.sinks, g.data_ptr(), beta.data_ptr(),
                                   stream_ptr(ab.device)), "bf_mem_gates")
    return qm, km, g, beta


def _new_ring(b, G, w, D, kdt, vdt, dev, overwritten: bool = False):
    """An empty ring (no valid slot). ``overwritten``: the caller's next write fills every slot before anything reads
    the ring (a prefill of at least W tokens from position 0), so the row tensors are left uninitialised; ring_pos
    still starts at -1 (no valid slot), so a call that fails before its write-back leaves a cache whose garbage
    rows are never read."""
    if overwritten:
        return dict(ring_k=torch.empty(b, G, w, D, dtype=kdt, device=dev),
                    ring_v=torch.empty(b, G, w, D, dtype=vdt, device=dev),
                    ring_km=torch.empty(b, w, G, D, dtype=torch.float32, device=dev),
                    ring_g=torch.empty(b, w, G, dtype=torch.float32, device=dev),
                    ring_beta=torch.empty(b, w, G, dtype=torch.float32, device=dev),
                    ring_pos=torch.full((w,), -1, dtype=torch.long, device=dev))
    return dict(ring_k=torch.zeros(b, G, w, D, dtype=kdt, device=dev),
                ring_v=torch.zeros(b, G, w, D, dtype=vdt, device=dev),
                ring_km=torch.zeros(b, w, G, D, dtype=torch.float32, device=dev),
                ring_g=torch.zeros(b, w, G, dtype=torch.float32, device=dev),
                ring_beta=torch.zeros(b, w, G, dtype=torch.float32, device=dev),
                ring_pos=torch.full((w,), -1, dtype=torch.long, device=dev))


def _ring_to(st: dict, kvdt: torch.dtype) -> None:
    """Bring the cache ring to the layouts the kernels read: ring_k / ring_v dense in the operand dtype, ring_km /
    ring_g / ring_beta dense fp32, ring_pos dense int64 (a cache written by the reference keeps the activations'
    dtype; the kernels write through these buffers in place, so they must match the dtype they are given)."""
    for key in ("ring_k", "ring_v"):
        if st[key].dtype != kvdt or not st[key].is_contiguous():
            st[key] = st[key].to(kvdt).contiguous()
    for key in ("ring_km", "ring_g", "ring_beta"):
        if st[key].dtype != torch.float32 or not st[key].is_contiguous():
            st[key] = st[key].float().contiguous()
    if st["ring_pos"].dtype != torch.long or not st["ring_pos"].is_contiguous():
        st["ring_pos"] = st["ring_pos"].long().contiguous()


def _decode(self, x, qr, kr, v, qm, km, g, beta, start, st, sink_k, sink_v, memory, zmix=None):
    """One token for every sequence: bf_decode_fwd (window, memory write on exit, read, mix, ring write). ``zmix``:
    the gamma logit mix(x) [B, H] fp32 if already computed."""
    c = self.c
    b = x.shape[0]
    H, G, D, w, r = c.h, c.hkv, c.dh, self.window, c.h // c.hkv
    dev = x.device
    kvdt = compute_dtype(kr, v)
    use_mem = memory and start + 1 > w
    S = None
    if use_mem:
        S = st.get("S")
        if S is None:
            S = torch.zeros(b, G, D, D, dtype=torch.float32, device=dev)
        elif not (S.dtype == torch.float32 and S.is_contiguous()):
            S = S.float().contiguous()
        st["S"] = S
    ns = 0 if sink_k is None else sink_k.size(2)
    sk = sink_k.to(kvdt).contiguous() if ns else None
    sv = sink_v.to(kvdt).contiguous() if ns else None
    _ring_to(st, kvdt)
    qrd = qr.to(torch.bfloat16 if qr.dtype == torch.bfloat16 else torch.float32).contiguous()
    z = None
    if use_mem:
        z = (zmix if zmix is not None else F.linear(x.float(), self.mix.weight.float(), self.mix.bias.float()))
        z = z.reshape(b, -1).contiguous()
    mix_lse = self.mix_lse.float().contiguous() if use_mem else None
    mem_scale = self.mem_scale.float().contiguous() if use_mem else None
    qm_ = qm.contiguous() if use_mem else None
    kr_, v_ = kr.to(kvdt).contiguous(), v.to(kvdt).contiguous()
    km_, g_, b_ = km.float().contiguous(), g.float().contiguous(), beta.float().contiguous()
    o = torch.empty(b, H, D, dtype=torch.float32, device=dev)
    lib = _lib.load()
    nbytes = _lib.ctypes.c_size_t(0)
    check(lib.bf_decode_workspace_size(b, G, r, D, w, _lib.ctypes.byref(nbytes)), "bf_decode_workspace_size")
    ws = workspace(nbytes.value, dev)
    ptr = lambda t_: t_.data_ptr() if t_ is not None else None
    check(lib.bf_decode_fwd(b, G, r, D, w, self.sinks, start, int(memory), dtype_code(kvdt), dtype_code(qrd.dtype),
                            ptr(qrd), ptr(qm_), ptr(kr_), ptr(v_), ptr(km_), ptr(g_), ptr(b_), ptr(z), ptr(mix_lse),
                            ptr(mem_scale), ptr(sk), ptr(sv), ns, ptr(st["ring_k"]), ptr(st["ring_v"]),
                            ptr(st["ring_km"]), ptr(st["ring_g"]), ptr(st["ring_beta"]), ptr(st["ring_pos"]), ptr(S),
                            ptr(o), None, ptr(ws), ws.numel(), stream_ptr(dev)), "bf_decode_fwd")
    return o.view(b, 1, H, D)


# Chunks of up to this many tokens over a cache run as consecutive decode steps. 1 (off): measured at B = 1, H = 24,
# G = 4, D = 256, W = 2048 + 4, a t = 2 chunk costs 207 us through the chunk kernels and 261 us as two decode steps,
# whose time is mostly host launch gaps between their six library calls.
SMALL_CHUNK = 1
BATCH_KEYS = ("sink_k", "sink_v", "ring_k", "ring_v", "ring_km", "ring_g", "ring_beta", "ring_pos", "S")


def new_batch_cache(self, b: int, dtype: torch.dtype, device) -> dict:
    """An empty per-sequence cache for ``student_batch``: the _student cache keys with one row per sequence and fixed
    sizes (the llama.cpp state-row model, ``bifrost.patch:221-239``): sink_k / sink_v [B, G, S, D] (rows 0 ..
    min(pos, S) - 1 present), ring_* as _student's, ring_pos [B, W] (-1 empty), S [B, G, D, D] zero."""
    c = self.c
    G, D, w, s = c.hkv, c.dh, self.window, self.sinks
    bc = _new_ring(b, G, w, D, dtype, dtype, device)
    bc["ring_pos"] = torch.full((b, w), -1, dtype=torch.long, device=device)
    bc["sink_k"] = torch.zeros(b, G, s, D, dtype=dtype, device=device)
    bc["sink_v"] = torch.zeros(b, G, s, D, dtype=dtype, device=device)
    bc["S"] = torch.zeros(b, G, D, D, dtype=torch.float32, device=device)
    return bc


def batch_cache_set(self, bc: dict, i: int, cache: Optional[dict]) -> None:
    """Row i of a batch cache := a single-sequence _student cache (B = 1; None or {} for an empty sequence)."""
    cache = cache or {}
    for key in BATCH_KEYS:
        bc[key][i].zero_() if key != "ring_pos" else bc[key][i].fill_(-1)
    if "ring_k" in cache:
        for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta"):
            bc[key][i].copy_(cache[key][0].to(bc[key].dtype))
        bc["ring_pos"][i].copy_(cache["ring_pos"])
    if cache.get("sink_k") is not None:
        n = cache["sink_k"].size(2)
        bc["sink_k"][i, :, :n].copy_(cache["sink_k"][0].to(bc["sink_k"].dtype))
        bc["sink_v"][i, :, :n].copy_(cache["sink_v"][0].to(bc["sink_v"].dtype))
    if cache.get("S") is not None:
        bc["S"][i].copy_(cache["S"][0])


def batch_cache_get(self, bc: dict, i: int, pos: int) -> dict:
    """Row i of a batch cache at position ``pos`` as a single-sequence _student cache (B = 1), the reverse of
    ``batch_cache_set``: sinks cut to the min(pos, S) present rows; S only once the memory has been written."""
    out = {key: bc[key][i:i + 1].clone() for key in ("ring_k", "ring_v", "ring_km", "ring_g", "ring_beta")}
    out["ring_pos"] = bc["ring_pos"][i].clone()
    n = min(pos, self.sinks)
    out["sink_k"] = bc["sink_k"][i:i + 1, :, :n].clone() if n else None
    out["sink_v"] = bc["sink_v"][i:i + 1, :, :n].clone() if n else None
    if pos > self.window:
        out["S"] = bc["S"][i:i + 1].clone()
    return out


def _fused_decode_ok(self, x, q, k, v, qr, kr) -> bool:
    """bf_student_decode covers this step: bf16 activations, a d_model the gate projection kernel takes, and the
    kernels' head limits."""
    c = self.c
    return (all(z_.dtype == torch.bfloat16 for z_ in (x, q, k, v, qr, kr)) and x.shape[-1] % 8 == 0
            and 2 * c.hkv + c.h <= 64 and c.h % c.hkv == 0 and c.h // c.hkv <= 8 and c.dh in (64, 128, 256))


def _student_decode(self, x, q, k, v, qr, kr, pos, pos_arr, st, sink_k, sink_v, ns, S, memory):
    """One bf_student_decode call (gate and memory projections, gates, decode step) for one token per sequence.
    pos_arr None: every sequence at ``pos`` with the cache of ``_student``; otherwise the batch cache of
    ``student_batch``. Returns o [B, 1, H, D] fp32."""
    c = self.c
    b = x.shape[0]
    H, G, D, w = c.h, c.hkv, c.dh, self.window
    dev = x.device
    xs = x.reshape(b, -1)
    if not xs.is_contiguous() or xs.data_ptr() % 16:
        xs = xs.contiguous()
    q_, k_, v_ = q.reshape(b, H, D).contiguous(), k.reshape(b, G, D).contiguous(), v.reshape(b, G, D).contiguous()
    qr_, kr_ = qr[:, :, 0].contiguous(), kr[:, :, 0].contiguous()
    f32 = lambda p_: p_.detach() if p_.dtype == torch.float32 and p_.is_contiguous() else p_.detach().float().contiguous()
    ab_b = None if self.ab.bias is None else f32(self.ab.bias)
    mix_b = None if self.mix.bias is None else f32(self.mix.bias)
    prm = (f32(self.fq), f32(self.fk), f32(self.ab.weight), ab_b, f32(self.mix.weight), mix_b, f32(self.A_log),
           f32(self.dt_bias), f32(self.decay_mask), f32(self.mix_lse), f32(self.mem_scale))
    o = torch.empty(b, H, D, dtype=torch.float32, device=dev)
    lib = _lib.load()
    nbytes = _lib.ctypes.c_size_t(0)
    check(lib.bf_student_decode_workspace_size(b, H, G, D, w, xs.shape[1], _lib.ctypes.byref(nbytes)),
          "bf_student_decode_workspace_size")
    ws = workspace(nbytes.value, dev)
    ptr = lambda t_: t_.data_ptr() if t_ is not None else None
    check(lib.bf_student_decode(b, H, G, D, w, self.sinks, pos, ptr(pos_arr), int(memory), xs.shape[1], ptr(xs),
                                ptr(q_), ptr(k_), ptr(v_), ptr(qr_), ptr(kr_), *(ptr(t_) for t_ in prm),
                                ptr(sink_k), ptr(sink_v), ns, ptr(st["ring_k"]), ptr(st["ring_v"]), ptr(st["ring_km"]),
                                ptr(st["ring_g"]), ptr(st["ring_beta"]), ptr(st["ring_pos"]), ptr(S), ptr(o), ptr(ws),
                                ws.numel(), stream_ptr(dev)), "bf_student_decode")
    return o.view(b, 1, H, D)


def student_batch(self, x, q, k, v, qr, kr, pos: torch.Tensor, cache: dict, memory: bool = True):
    """One token for each of B sequences at its own position (continuous batching; llama.cpp's multi-sequence ubatch,
    ``bifrost.patch:841-884``): per sequence the result and the cache update of ``_student`` with t == 1
    (``hibrit.py:363-424``) on that sequence's own cache, in one bf_decode_fwd_batch call.

    x [B, 1, d]; q [B, 1, H, D]; k, v [B, 1, G, D]; qr [B, H, 1, D], kr [B, G, 1, D]; pos [B] int64 on the device;
    cache: a batch cache (``new_batch_cache``), mutated in place. Returns o [B, 1, H, D] fp32."""
    require_device(x, q, k, v, qr, kr, pos)
    require_no_grad(x, q, k, v, qr, kr)
    c = self.c
    b = x.shape[0]
    if x.shape[1] != 1:
        raise BifrostError("student_batch takes one token per sequence")
    H, G, D, w, r = c.h, c.hkv, c.dh, self.window, c.h // c.hkv
    dev = x.device
    kvdt = cache["ring_k"].dtype
    pos = pos.to(device=dev, dtype=torch.long).contiguous()
    if kvdt == torch.bfloat16 and _fused_decode_ok(self, x, q, k, v, qr, kr):
        return _student_decode(self, x, q, k, v, qr, kr, 0, pos, cache, cache["sink_k"], cache["sink_v"],
                               self.sinks, cache["S"], memory)
    # memory inputs without the sink mask of beta (position S passed), then the mask per sequence
    if all(z_.dtype == torch.bfloat16 for z_ in (q, k, qr, kr)):
        ab, z = _gate_logits(self, x)
        qm, km, g, beta = _mem_inputs_bf16(self, ab, q, k, self.sinks, torch.float32)
    else:
        qm, km, g, beta = self._mem_inputs(x, q, k, torch.full((1,), self.sinks, device=dev))
        z = F.linear(x.float(), self.mix.weight.float(), self.mix.bias.float())
    beta = beta * (pos >= self.sinks).float()[:, None, None]
    z = z.reshape(b, H).contiguous()
    f32 = lambda t_: t_.float().contiguous()
    qm_, km_, g_, b_ = f32(qm[:, 0]), f32(km[:, 0]), f32(g[:, 0]), f32(beta[:, 0])
    qrd = qr[:, :, 0].to(torch.bfloat16 if qr.dtype == torch.bfloat16 else torch.float32).contiguous()
    kr_, v_ = kr[:, :, 0].to(kvdt).contiguous(), v[:, 0].to(kvdt).contiguous()
    mix_lse, mem_scale = self.mix_lse.float().contiguous(), self.mem_scale.float().contiguous()
    o = torch.empty(b, H, D, dtype=torch.float32, device=dev)
    lib = _lib.load()
    nbytes = _lib.ctypes.c_size_t(0)
    check(lib.bf_decode_workspace_size(b, G, r, D, w, _lib.ctypes.byref(nbytes)), "bf_decode_workspace_size")
    ws = workspace(nbytes.value, dev)
    ptr = lambda t_: t_.data_ptr()
    check(lib.bf_decode_fwd_batch(b, G, r, D, w, self.sinks, ptr(pos), int(memory), dtype_code(kvdt),
                                  dtype_code(qrd.dtype), ptr(qrd), ptr(qm_), ptr(kr_), ptr(v_), ptr(km_), ptr(g_),
                                  ptr(b_), ptr(z), ptr(mix_lse), ptr(mem_scale), ptr(cache["sink_k"]),
                                  ptr(cache["sink_v"]), ptr(cache["ring_k"]), ptr(cache["ring_v"]),
                                  ptr(cache["ring_km"]), ptr(cache["ring_g"]), ptr(cache["ring_beta"]),
                                  ptr(cache["ring_pos"]), ptr(cache["S"]), ptr(o), None, ptr(ws), ws.numel(),
                                  stream_ptr(dev)), "bf_decode_fwd_batch")
    return o.view(b, 1, H, D)


def student(self, x, q, k, v, qr, kr, start: int, cache: Optional[dict], memory: bool = True):
    """Window + sinks attention, delta-rule memory written on window exit, gamma mix (``hibrit.py:363-424``).

    x [B, t, d]; q [B, t, H, D] (normed, pre-RoPE); k, v [B, t, G, D]; qr [B, H, t, D], kr [B, G, t, D] (RoPE'd).
    cache: dict mutated in place (the reference's keys and shapes) or None. Returns o [B, t, H, D] fp32.

    With autograd recording and a trainable new parameter (or a memory input that requires grad), as in the
    conversion's stage A (``distill_pair``, ``hibrit.py:434-439``), the call is differentiable: see
    ``_student_autograd``.
    """
    require_device(x, q, k, v, qr, kr)
    if _needs_grad(self, x, q, k, v, qr, kr):
        return _student_autograd(self, x, q, k, v, qr, kr, start, cache, memory)
    c = self.c
    b, t = x.shape[:2]
    w, s = self.window, self.sinks
    dev = x.device
    st = cache if cache is not None else {}
    if 1 < t <= SMALL_CHUNK and "ring_k" in st:
        # a few tokens over a cache (an MTP verification, hibrit.py:758): one decode step each, the reference's
        # chunking invariance (a chunk equals its tokens one at a time); a decode step splits the window over
        # the chip, where the chunk kernels would run one workgroup per query head
        return torch.cat([student(self, *(z[:, i:i + 1] for z in (x, q, k, v)), qr[:, :, i:i + 1], kr[:, :, i:i + 1],
                                  start + i, st, memory) for i in range(t)], 1)
    vt = v.transpose(1, 2)
    sink_k, sink_v = st.get("sink_k"), st.get("sink_v")
    n_new = max(0, min(t, s - start))
    if n_new:
        # stored dense: a view of the chunk would keep the whole chunk alive in the cache and be copied to a dense
        # operand by every later call (two small copy launches per chunk call)
        sink_k = kr[:, :, :n_new].contiguous() if sink_k is None else torch.cat((sink_k, kr[:, :, :n_new]), 2)
        sink_v = vt[:, :, :n_new].contiguous() if sink_v is None else torch.cat((sink_v, vt[:, :, :n_new]), 2)
    if t == 1 and _fused_decode_ok(self, x, q, k, v, qr, kr):
        if "ring_k" not in st:
            st.update(_new_ring(b, c.hkv, w, c.dh, torch.bfloat16, torch.bfloat16, dev))
        _ring_to(st, torch.bfloat16)
        S = None
        if memory and start + 1 > w:
            S = st.get("S")
            if S is None:
                S = torch.zeros(b, c.hkv, c.dh, c.dh, dtype=torch.float32, device=dev)
            elif not (S.dtype == torch.float32 and S.is_contiguous()):
                S = S.float().contiguous()
            st["S"] = S
        ns = 0 if sink_k is None else sink_k.size(2)
        sk = sink_k.to(torch.bfloat16).contiguous() if ns else None
        sv = sink_v.to(torch.bfloat16).contiguous() if ns else None
        o = _student_decode(self, x, q, k, v, qr, kr, start, None, st, sk, sv, ns, S, memory)
        st["sink_k"], st["sink_v"] = sink_k, sink_v
        return o
    zmix = None
    if all(z.dtype == torch.bfloat16 for z in (q, k, qr, kr)):
        # fused: the gate projections, qm / km (bf16 for a chunk's memory branch, fp32 for the decode step), gates
        ab, zmix = _gate_logits(self, x)
        qm, km, g, beta = _mem_inputs_bf16(self, ab, q, k, start, torch.bfloat16 if t > 1 else torch.float32)
    else:
        qm, km, g, beta = self._mem_inputs(x, q, k, torch.arange(start, start + t, device=dev))
    if "ring_k" not in st:
        # a prefill of t >= W tokens from position 0 writes every ring slot (bf_layer_prefill_fwd's write-back) and
        # reads none before that
        full = t >= w and start == 0
        st.update(_new_ring(b, c.hkv, w, c.dh, kr.dtype, vt.dtype, dev, overwritten=full))
    if t == 1:
        o = _decode(self, x, qr, kr[:, :, 0], v[:, 0], qm[:, 0], km[:, 0], g[:, 0], beta[:, 0], start, st, sink_k,
                    sink_v, memory, zmix)
    else:
        o = _prefill(self, x, qr, kr, v, qm, km, g, beta, start, st, sink_k, sink_v, memory, zmix)
    st["sink_k"], st["sink_v"] = sink_k, sink_v
    return o


def _new_params(self):
    """The trainable tensors of the conversion (``NEW``): fq, fk, ab, mix, mix_lse, mem_scale, A_log, dt_bias."""
    out = []
    for n in NEW:
        p = getattr(self, n, None)
        if isinstance(p, nn.Module):
            out.extend(p.parameters())
        elif p is not None:
            out.append(p)
    return out


def _needs_grad(self, *inputs) -> bool:
    return torch.is_grad_enabled() and (any(t_ is not None and t_.requires_grad for t_ in inputs) or
                                        any(p.requires_grad for p in _new_params(self)))


def _window_lse(self, qr, kr, v, start, st, sink_k, sink_v):
    """Window + sinks attention with the per-row LSE and no mix (``hibrit.py:336-361``): bf_window_fwd over the chunk
    and, for positions before ``start``, the cache ring ``st`` (if it has one). Returns (o_win [B, t, H, D] fp32,
    lse [B, H, t] fp32); no autograd graph (the window branch has no trainable parameter)."""
    c = self.c
    b, t = qr.shape[0], qr.shape[2]
    H, G, D, w, r = c.h, c.hkv, c.dh, self.window, c.h // c.hkv
    dev = qr.device
    cdt = compute_dtype(qr, kr, v)
    ring = "ring_k" in st
    if ring:
        _ring_to(st, cdt)
    unit = lambda t_: t_ if t_.stride(-1) == 1 else t_.contiguous()
    q_, k_, v_ = (unit(z.detach().to(cdt)) for z in (qr, kr, v))
    ns = 0 if sink_k is None else sink_k.size(2)
    sk = sink_k.detach().to(cdt).contiguous() if ns else None
    sv = sink_v.detach().to(cdt).contiguous() if ns else None
    o = torch.empty(b, t, H, D, dtype=torch.float32, device=dev)
    lse = torch.empty(b, H, t, dtype=torch.float32, device=dev)
    ptr = lambda t_: t_.data_ptr() if t_ is not None else None
    check(_lib.load().bf_window_fwd(
        b, G, r, D, t, w, self.sinks, start, dtype_code(cdt), ptr(q_), *_strides(q_, (0, 1, 2)), ptr(k_),
        *_strides(k_, (0, 1, 2)), ptr(v_), *_strides(v_, (0, 2, 1)), ptr(st["ring_k"]) if ring else None,
        ptr(st["ring_v"]) if ring else None, ptr(st["ring_pos"]) if ring else None, ptr(sk), ptr(sv), ns, 0, None, 0,
        None, None, None, ptr(o), _lib.DTYPE_F32, ptr(lse), stream_ptr(dev)), "bf_window_fwd")
    return o, lse


def _student_autograd(self, x, q, k, v, qr, kr, start: int, cache: Optional[dict], memory: bool = True):
    """``_student`` with gradients, for the conversion's training (stage A, ``distill_pair``, ``hibrit.py:434-439``):
    the memory inputs (``_mem_inputs``), the write stream, the gamma mix and the cache update are PyTorch ops on the
    GPU and the delta rule is ``motor.delta_rule_gqa`` (``bf_gdn_fwd`` forward, ``bf_gdn_bwd`` backward, fp32), so the
    gradients of the new parameters (and of q, k, x) are those of the reference's autograd graph. The window branch
    (``bf_window_fwd``) has no trainable parameter and its output and LSE enter as constants: qr, kr and v must not
    require grad (in the reference's training they come from frozen projections, ``hibrit.py:556-561``)."""
    from .motor import delta_rule_gqa
    if any(t_.requires_grad for t_ in (qr, kr, v)):
        raise BifrostError("the window branch has no backward: qr, kr and v must not require grad (the conversion "
                           "trains only the new parameters; the projections are frozen)")
    c = self.c
    b, t = x.shape[:2]
    H, G, D, w, s, r = c.h, c.hkv, c.dh, self.window, self.sinks, c.h // c.hkv
    dev = x.device
    st = cache if cache is not None else {}
    pos = torch.arange(start, start + t, device=dev)
    vt = v.transpose(1, 2)
    sink_k, sink_v = st.get("sink_k"), st.get("sink_v")
    n_new = max(0, min(t, s - start))
    if n_new:
        sink_k = kr[:, :, :n_new] if sink_k is None else torch.cat((sink_k, kr[:, :, :n_new]), 2)
        sink_v = vt[:, :, :n_new] if sink_v is None else torch.cat((sink_v, vt[:, :, :n_new]), 2)
    o_win, lse = _window_lse(self, qr, kr, v, start, st, sink_k, sink_v)
    o = o_win
    use_mem = memory and start + t > w
    if use_mem or cache is not None:
        qm, km, g, beta = self._mem_inputs(x, q, k, pos)
    if use_mem:
        s0 = st.get("S")
        ring = "ring_k" in st
        if start == 0 and s0 is None and not ring:
            # empty history: the first W writes are empty (g = beta = 0) and the queries before W have gamma = 0, so
            # the queries W .. t-1 read the state after the writes of tokens 0 .. t-W-1
            o_tail, sm = delta_rule_gqa(qm[:, w:].reshape(b, t - w, G, r, D), km[:, :t - w], v[:, :t - w].float(),
                                        g[:, :t - w], beta[:, :t - w], 64, None)
            o_mem = torch.cat((o_tail.new_zeros(b, w, G, r, D), o_tail), 1).reshape(b, t, H, D)
        else:
            # token i - W is written before the query at position i reads: the stream is [ring ; chunk][:t]
            pp = torch.arange(start - w, start, device=dev)
            if ring:
                idx = pp % w
                rv = st["ring_v"][:, :, idx].transpose(1, 2).float()
                rkm, rg, rb = st["ring_km"][:, idx].float(), st["ring_g"][:, idx].float(), st["ring_beta"][:, idx].float()
                vf = (st["ring_pos"][idx] == pp).float()[None, :, None]
            else:
                rv = torch.zeros(b, w, G, D, device=dev)
                rkm, rg, rb = torch.zeros_like(rv), torch.zeros(b, w, G, device=dev), torch.zeros(b, w, G, device=dev)
                vf = torch.zeros(1, w, 1, device=dev)
            wk = torch.cat((rkm, km.float()), 1)[:, :t]
            wv = torch.cat((rv, v.float()), 1)[:, :t]
            wg = torch.cat((rg * vf, g), 1)[:, :t]
            wb = torch.cat((rb * vf, beta), 1)[:, :t]
            o_mem, sm = delta_rule_gqa(qm.reshape(b, t, G, r, D), wk, wv, wg, wb, 64, s0)
            o_mem = o_mem.reshape(b, t, H, D)
        z = F.linear(x.float(), self.mix.weight.float(), self.mix.bias.float())
        gamma = torch.sigmoid(z + self.mix_lse.float() * (lse.transpose(1, 2) - math.log(w)))
        gamma = gamma * (pos >= w).float()[None, :, None]
        o = o_win + gamma[..., None] * (self.mem_scale.float()[:, None] * o_mem - o_win)
        if cache is not None:
            cache["S"] = sm
    if cache is not None:
        if "ring_k" not in cache:
            cache.update(_new_ring(b, G, w, D, compute_dtype(qr, kr, v), compute_dtype(qr, kr, v), dev))
        m_ = min(t, w)
        slot = pos[-m_:] % w
        with torch.no_grad():
            cache["ring_k"][:, :, slot] = kr[:, :, -m_:].to(cache["ring_k"].dtype)
            cache["ring_v"][:, :, slot] = vt[:, :, -m_:].to(cache["ring_v"].dtype)
            cache["ring_pos"][slot] = pos[-m_:]
        # recorded by autograd, as the reference's slot assignments are (hibrit.py:419-420): a later chunk that reads
        # these rows back into its write stream carries their gradient to fk, ab, A_log and dt_bias
        cache["ring_km"][:, slot], cache["ring_g"][:, slot] = km[:, -m_:].float(), g[:, -m_:].float()
        cache["ring_beta"][:, slot] = beta[:, -m_:].float()
        cache["sink_k"], cache["sink_v"] = sink_k, sink_v
    return o


def window(self, qr, ext_k, ext_v, ext_pos, sink_k, sink_v, pos):
    """``HybridAttention._window`` (``hibrit.py:336-361``) on ``bf_window_fwd``: qr [B, H, t, D]; ext_k / ext_v
    [B, G, W + t, D] = [the ring positions start - W .. start - 1 in time order ; the chunk]; ext_pos [W + t] (-1 for
    an empty ring entry, else the position, and the chunk's positions start .. start + t - 1); sink_k / sink_v
    [B, G, ns, D] or None; pos [t] = start .. start + t - 1. Returns (o_win [B, t, H, D] fp32, lse [B, H, t] fp32).

    The kernel reads history from a ring indexed by position mod W, so the first W entries are rotated into that
    order (position p = start - W + j goes to slot p mod W = (start + j) mod W); one host read of ``pos[0]``."""
    dev = require_device(qr, ext_k, ext_v, ext_pos, pos)
    require_no_grad(qr, ext_k, ext_v)
    w = self.window
    start = int(pos[0].item())
    t = qr.shape[2]
    if ext_k.shape[2] != w + t or ext_pos.numel() != w + t or pos.numel() != t:
        raise BifrostError("ext_k / ext_v / ext_pos must hold W ring entries followed by the chunk")
    sh = start % w
    st = {"ring_k": torch.roll(ext_k[:, :, :w], sh, 2), "ring_v": torch.roll(ext_v[:, :, :w], sh, 2),
          "ring_pos": torch.roll(ext_pos[:w].to(device=dev, dtype=torch.long), sh, 0).contiguous(),
          "ring_km": torch.empty(0, device=dev), "ring_g": torch.empty(0, device=dev),
          "ring_beta": torch.empty(0, device=dev)}
    kr, vt = ext_k[:, :, w:], ext_v[:, :, w:]
    return _window_lse(self, qr, kr, vt.transpose(1, 2), start, st, sink_k, sink_v)


def _strides(t: torch.Tensor, dims):
    return tuple(int(t.stride(d)) for d in dims)


def _prefill(self, x, qr, kr, v, qm, km, g, beta, start, st, sink_k, sink_v, memory, zmix=None):
    """A chunk of t > 1 tokens in one bf_layer_prefill_fwd call: the delta-rule memory on the write stream (ring rows
    leaving the window, then the chunk's own rows, hibrit.py:391-408), the window + sinks + LSE with the gamma mix
    (hibrit.py:385-411), then the ring / state write-back (hibrit.py:412-423). From an empty cache (start 0, no
    state) the queries before W never read the memory, so the library runs the memory on queries W..t-1 against the
    writes of tokens 0..t-W-1 only. ``zmix``: the gamma logit mix(x) [B, t, H] fp32 if already computed."""
    c = self.c
    b, t = x.shape[:2]
    H, G, D, w, r = c.h, c.hkv, c.dh, self.window, c.h // c.hkv
    dev = x.device
    cdt = compute_dtype(qr, kr, v)
    lib = _lib.load()
    use_mem = memory and start + t > w
    _ring_to(st, cdt)
    S, valid = st.get("S"), 1
    if S is None:
        S, valid = torch.empty(b, G, D, D, dtype=torch.float32, device=dev), 0
    elif not (S.dtype == torch.float32 and S.is_contiguous()):
        S = S.float().contiguous()
    z = mix_lse = mem_scale = None
    if use_mem:
        z = zmix if zmix is not None else F.linear(x.float(), self.mix.weight.float(), self.mix.bias.float())
        z = z.contiguous()
        mix_lse = self.mix_lse.float().contiguous()
        mem_scale = self.mem_scale.float().contiguous()
    mdt = lambda t_: t_.contiguous() if t_.dtype in (torch.float32, torch.bfloat16) else t_.to(cdt).contiguous()
    qm_, km_ = mdt(qm), mdt(km)
    g_, b_ = g.float().contiguous(), beta.float().contiguous()
    unit = lambda t_: t_ if t_.stride(-1) == 1 else t_.contiguous()
    q_, k_, v_ = unit(qr.to(cdt)), unit(kr.to(cdt)), unit(v.to(cdt))
    ns = 0 if sink_k is None else sink_k.size(2)
    sk = sink_k.to(cdt).contiguous() if ns else None
    sv = sink_v.to(cdt).contiguous() if ns else None
    o = torch.empty(b, t, H, D, dtype=torch.float32, device=dev)
    nbytes = _lib.ctypes.c_size_t(0)
    check(lib.bf_layer_prefill_workspace_size(b, G, r, D, t, dtype_code(cdt), _lib.ctypes.byref(nbytes)),
          "bf_layer_prefill_workspace_size")
    ws = workspace(nbytes.value, dev)
    ptr = lambda t_: t_.data_ptr() if t_ is not None else None
    check(lib.bf_layer_prefill_fwd(
        b, G, r, D, t, w, self.sinks, start, int(memory), dtype_code(cdt),
        ptr(q_), *_strides(q_, (0, 1, 2)), ptr(k_), *_strides(k_, (0, 1, 2)), ptr(v_), *_strides(v_, (0, 2, 1)),
        ptr(qm_), dtype_code(qm_.dtype), ptr(km_), dtype_code(km_.dtype), ptr(g_), ptr(b_), ptr(z), ptr(mix_lse),
        ptr(mem_scale), ptr(sk), ptr(sv), ns, ptr(st["ring_k"]), ptr(st["ring_v"]), ptr(st["ring_km"]),
        ptr(st["ring_g"]), ptr(st["ring_beta"]), ptr(st["ring_pos"]), ptr(S), valid, ptr(o), None, ptr(ws),
        ws.numel(), stream_ptr(dev)), "bf_layer_prefill_fwd")
    if use_mem:
        st["S"] = S
    return o


class BifrostCore(nn.Module):
    """The converted layer's new parameters and student path, with the reference's attribute names.

    Holds ``fq [H,D,D], fk [G,D,D], ab (Linear d -> 2G), mix (Linear d -> H), mix_lse [H], mem_scale [H], A_log [G],
    dt_bias [G]`` and the buffer ``decay_mask [G]``; ``window`` and ``sinks`` are set by ``convert``.
    """

    def __init__(self, c: CoreConfig):
        super().__init__()
        self.c = c
        self.converted = False

    def convert(self, window: int, sinks: int, archival: int, mem_init: str = "long") -> None:
        """Conversion init (``hibrit.py:211-240``): identity fq/fk, zero gates with mix bias -2, dt ~ logU[1e-3, 1e-1],
        "long" memory: read scale sqrt(D), decay half-lives logspace(log10 W, 6, G) tokens, first ``archival`` KV
        heads never decay; "mamba": read scale 1, A in U[1, 16]."""
        c = self.c
        dev = next((p.device for p in self.parameters()), torch.device("cpu"))
        self.window, self.sinks = window, sinks
        self.fq = nn.Parameter(torch.eye(c.dh, device=dev).repeat(c.h, 1, 1))
        self.fk = nn.Parameter(torch.eye(c.dh, device=dev).repeat(c.hkv, 1, 1))
        self.ab = nn.Linear(c.d, 2 * c.hkv, device=dev)
        self.mix = nn.Linear(c.d, c.h, device=dev)
        for lin in (self.ab, self.mix):
            nn.init.zeros_(lin.weight)
            nn.init.zeros_(lin.bias)
        nn.init.constant_(self.mix.bias, -2.0)
        self.mix_lse = nn.Parameter(torch.zeros(c.h, device=dev))
        dt = torch.exp(torch.empty(c.hkv, device=dev).uniform_(math.log(1e-3), math.log(1e-1)))
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        if mem_init == "mamba":
            self.mem_scale = nn.Parameter(torch.ones(c.h, device=dev))
            self.A_log = nn.Parameter(torch.empty(c.hkv, device=dev).uniform_(1.0, 16.0).log())
        else:
            self.mem_scale = nn.Parameter(torch.full((c.h,), float(c.dh) ** 0.5, device=dev))
            life = torch.logspace(math.log10(max(window, 2)), 6.0, c.hkv, device=dev)
            self.A_log = nn.Parameter((math.log(2.0) / (life * dt)).log())
        mask = torch.ones(c.hkv, device=dev)
        mask[:archival] = 0.0
        self.register_buffer("decay_mask", mask, persistent=False)
        self.converted = True

    _mem_inputs = mem_inputs
    _window = window
    _student = student
    _teacher = teacher
    set_retrieval = set_retrieval

    def forward(self, x, q, k, v, qr, kr, start: int = 0, cache: Optional[dict] = None, memory: bool = True):
        return self._student(x, q, k, v, qr, kr, start, cache, memory)
