"""Formats around the converted layer: the llama.cpp state row of a sequence and the GGUF tensors of a conversion.

- ``pack_llama_state`` / ``unpack_llama_state`` (``bf_llama_state_pack`` / ``bf_llama_state_unpack``): the student
  cache of ``heimdall_amd.hibrit`` (the reference's ``_student`` cache: ``sink_k, sink_v, ring_k, ring_v, ring_km,
  ring_g, ring_beta, ring_pos, S``) <-> the per-sequence recurrent row of a Bifrost layer in the patched llama.cpp
  (``Heimdall/llamacpp/bifrost.patch:221-239,816-827,1000-1013``), on the GPU, so sequences can move between a
  llama.cpp build and these kernels.
- ``gguf_tensors`` / ``load_gguf_tensors``: a ``BifrostCore``'s conversion parameters <-> the
  ``blk.N.bifrost_*`` tensors that ``Heimdall/llamacpp/bifrost_gguf.py:24-47`` writes, and the GGUF keys
  (``<arch>.bifrost.window / sinks / layers``).
- ``conversion_state`` / ``apply_conversion``: the conversion dict of ``HybridLM.conversion_state`` /
  ``apply_conversion`` (``Heimdall/heimdall/hibrit.py:780-800``) for a set of ``BifrostCore`` layers.
"""
import ctypes
from typing import Dict, Optional

import torch

from . import _lib
from ._device import BifrostError, check, dtype_code, require_device, stream_ptr

NEW = ("fq", "fk", "ab", "mix", "mix_lse", "mem_scale", "A_log", "dt_bias")


def llama_state_floats(G: int, D: int, W: int, S: int) -> int:
    """Floats of one sequence's row: ceil((S + W + 2) / 32) * 32 * (5 G D + 2 G) + D^2 G."""
    out = ctypes.c_int64(0)
    check(_lib.load().bf_llama_state_floats(G, D, W, S, ctypes.byref(out)), "bf_llama_state_floats")
    return out.value


def pack_llama_state(cache: dict, n: int, W: int, S: int) -> torch.Tensor:
    """rows [B, llama_state_floats] f32 from a student cache after n tokens (window W, S sinks)."""
    rk, rv = cache["ring_k"], cache["ring_v"]
    dev = require_device(rk, rv, cache["S"])
    B, G, W_, D = rk.shape
    if W_ != W or rv.dtype != rk.dtype:
        raise BifrostError(f"ring_k must be [B, G, {W}, D] with ring_v of the same dtype")
    sk, sv = cache.get("sink_k"), cache.get("sink_v")
    ns = 0 if sk is None else sk.shape[2]
    c = lambda t: t.contiguous() if t is not None else None
    rows = torch.empty(B, llama_state_floats(G, D, W, S), dtype=torch.float32, device=dev)
    ptr = lambda t: t.data_ptr() if t is not None else None
    sk, sv = c(sk.to(rk.dtype)) if ns else None, c(sv.to(rk.dtype)) if ns else None
    check(_lib.load().bf_llama_state_pack(
        B, G, D, W, S, int(n), dtype_code(rk.dtype), c(rk).data_ptr(), c(rv).data_ptr(),
        c(cache["ring_km"].float()).data_ptr(), c(cache["ring_g"].float()).data_ptr(),
        c(cache["ring_beta"].float()).data_ptr(), c(cache["ring_pos"].long()).data_ptr(), ptr(sk), ptr(sv), ns,
        c(cache["S"].float()).data_ptr(), rows.data_ptr(), stream_ptr(dev)), "bf_llama_state_pack")
    return rows


def unpack_llama_state(rows: torch.Tensor, n: int, W: int, S: int, G: int, D: int,
                       kv_dtype: torch.dtype = torch.float32) -> dict:
    """The student cache from rows [B, llama_state_floats] after n tokens: ring entries for positions
    max(0, n - W) .. n - 1, min(S, n) sinks, the state; k / v in ``kv_dtype``."""
    dev = require_device(rows)
    B = rows.shape[0]
    if rows.shape[1] != llama_state_floats(G, D, W, S) or rows.dtype != torch.float32:
        raise BifrostError("rows must be [B, llama_state_floats(G, D, W, S)] float32")
    ns = min(S, int(n))
    e = lambda *s, dt=torch.float32: torch.empty(*s, dtype=dt, device=dev)
    out = dict(ring_k=e(B, G, W, D, dt=kv_dtype), ring_v=e(B, G, W, D, dt=kv_dtype), ring_km=e(B, W, G, D),
               ring_g=e(B, W, G), ring_beta=e(B, W, G), ring_pos=e(W, dt=torch.int64), S=e(B, G, D, D))
    sk = e(B, G, ns, D, dt=kv_dtype) if ns else None
    sv = e(B, G, ns, D, dt=kv_dtype) if ns else None
    r = rows.contiguous()
    check(_lib.load().bf_llama_state_unpack(
        B, G, D, W, S, int(n), dtype_code(kv_dtype), r.data_ptr(), out["ring_k"].data_ptr(), out["ring_v"].data_ptr(),
        out["ring_km"].data_ptr(), out["ring_g"].data_ptr(), out["ring_beta"].data_ptr(), out["ring_pos"].data_ptr(),
        sk.data_ptr() if ns else None, sv.data_ptr() if ns else None, ns, out["S"].data_ptr(), stream_ptr(dev)),
        "bf_llama_state_unpack")
    out["sink_k"], out["sink_v"] = sk, sv
    return out


# ---------------------------------------------------------------------------------------------- GGUF tensors
def gguf_tensors(core, layer: int) -> Dict[str, torch.Tensor]:
    """``blk.<layer>.bifrost_*`` float32 CPU tensors of a converted core (``bifrost_gguf.py:24-47``): fq / fk
    transposed per head (ggml's mul_mat contracts the first axis), a = -e^A_log with the archival heads (decay_mask
    0) zeroed, ab / mix split into weight and bias, mix_lse, mem_scale, dt = dt_bias."""
    f = lambda t: t.detach().float().cpu().contiguous()
    p = f"blk.{layer}."
    return {p + "bifrost_fq": f(core.fq.transpose(1, 2)), p + "bifrost_fk": f(core.fk.transpose(1, 2)),
            p + "bifrost_ab": f(core.ab.weight), p + "bifrost_ab_b": f(core.ab.bias),
            p + "bifrost_mix": f(core.mix.weight), p + "bifrost_mix_b": f(core.mix.bias),
            p + "bifrost_mix_lse": f(core.mix_lse), p + "bifrost_mem_scale": f(core.mem_scale),
            p + "bifrost_a": f(-core.A_log.exp() * core.decay_mask), p + "bifrost_dt": f(core.dt_bias)}


def gguf_metadata(arch: str, window: int, sinks: int, converted_layers, n_layers: int) -> dict:
    """The GGUF keys the patched llama.cpp reads: ``<arch>.bifrost.window``, ``.sinks`` and ``.layers`` (one 0 / 1
    per block)."""
    conv = set(converted_layers)
    return {f"{arch}.bifrost.window": int(window), f"{arch}.bifrost.sinks": int(sinks),
            f"{arch}.bifrost.layers": [1 if i in conv else 0 for i in range(n_layers)]}


def load_gguf_tensors(core, tensors: Dict[str, torch.Tensor], layer: int, window: int, sinks: int) -> None:
    """Set a core's conversion from ``blk.<layer>.bifrost_*`` tensors. The archival heads are those with a == 0
    (their A_log is not stored; it is set to 0, which their decay mask of 0 makes irrelevant)."""
    p = f"blk.{layer}."
    t = lambda k: tensors[p + k].float()
    a = t("bifrost_a")
    archival = int((a == 0).sum())
    if archival and not bool((a[:archival] == 0).all()):
        raise BifrostError("archival heads must be the first KV heads (a == 0)")
    core.convert(window, sinks, archival)
    dev = core.fq.device
    with torch.no_grad():
        core.fq.copy_(t("bifrost_fq").transpose(1, 2).to(dev))
        core.fk.copy_(t("bifrost_fk").transpose(1, 2).to(dev))
        core.ab.weight.copy_(t("bifrost_ab").to(dev))
        core.ab.bias.copy_(t("bifrost_ab_b").to(dev))
        core.mix.weight.copy_(t("bifrost_mix").to(dev))
        core.mix.bias.copy_(t("bifrost_mix_b").to(dev))
        core.mix_lse.copy_(t("bifrost_mix_lse").to(dev))
        core.mem_scale.copy_(t("bifrost_mem_scale").to(dev))
        core.A_log.copy_(torch.where(a != 0, (-a).clamp_min(1e-38).log(), torch.zeros_like(a)).to(dev))
        core.dt_bias.copy_(t("bifrost_dt").to(dev))


# ---------------------------------------------------------------------------------------------- conversion dict
def conversion_state(cores: Dict[str, object], meta: Optional[dict] = None) -> dict:
    """``{"conv": [{name, window, sinks, archival}], "params": {"<name>.self_attn.<param>": fp32 CPU}}`` for the
    converted cores, keyed by layer name as ``HybridLM.conversion_state`` does (``hibrit.py:780-788``)."""
    conv, params = [], {}
    for name, core in cores.items():
        if not getattr(core, "converted", False):
            continue
        conv.append(dict(name=name, window=core.window, sinks=core.sinks,
                         archival=int((core.decay_mask == 0).sum())))
        for n, p in core.named_parameters():
            if n.split(".")[0] in NEW:
                params[f"{name}.self_attn.{n}"] = p.detach().float().cpu()
    return {"conv": conv, "params": params, "meta": meta or {}}


def apply_conversion(cores: Dict[str, object], state: dict) -> None:
    """Convert and load the cores named in a conversion dict (``HybridLM.apply_conversion``, ``hibrit.py:790-800``)."""
    for cv in state["conv"]:
        if cv["name"] in cores:
            cores[cv["name"]].convert(cv["window"], cv["sinks"], cv["archival"])
    for name, core in cores.items():
        own = dict(core.named_parameters())
        prefix = f"{name}.self_attn."
        with torch.no_grad():
            for k, t in state["params"].items():
                if k.startswith(prefix) and k[len(prefix):] in own:
                    own[k[len(prefix):]].copy_(t.to(own[k[len(prefix):]].device))
