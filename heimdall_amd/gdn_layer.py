"""The native Gated DeltaNet layer on the GPU (reference: ``GatedDeltaNet``, ``Heimdall/heimdall/hibrit.py:136-184``).

``GatedDeltaNet`` keeps the reference module's parameter names (``in_proj_qkv``, ``in_proj_z``, ``in_proj_b``,
``in_proj_a``, ``conv1d.weight``, ``dt_bias``, ``A_log``, ``norm.weight``, ``out_proj``), so a state dict loads
unchanged, and its ``forward(x, cache=None, start=0)`` with the same cache keys ("conv": the last K - 1 rows of
in_proj_qkv(x), "S": the fp32 state per value head). The frozen projections stay PyTorch matrix products; between
them three library calls do the work:

- ``conv_inputs`` (``bf_gdn_conv_inputs``): causal conv + SiLU + l2norm + q scale + head repeat + beta / g gates;
- the delta rule (``bf_gdn_fwd`` for a chunk, ``bf_gdn_step`` for one token with a carried state);
- ``gated_norm`` (``bf_gated_norm``): weight * RMSNorm(o) * SiLU(z).

``gdn_layer_packed`` runs the same core on packed variable-length sequences (``cu_seqlens``), each sequence
independent with its own conv prefix and state.
"""
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from ._device import (BifrostError, check, dtype_code, gdn_forward, require_device, require_no_grad, stream_ptr)
from .kernels import gdn_step


@dataclass
class GdnLayerConfig:
    """The fields of ``HybridConfig`` the layer reads (``hibrit.py:91-94``)."""
    d: int
    lin_hk: int
    lin_hv: int
    lin_dk: int
    lin_dv: int
    conv_k: int = 4
    eps: float = 1e-6


def _seqlens(num_seqs: int, seq_len: int, dev) -> torch.Tensor:
    return torch.arange(0, (num_seqs + 1) * seq_len, seq_len, dtype=torch.int32, device=dev)


def conv_inputs(z: torch.Tensor, conv_w: torch.Tensor, prefix: Optional[torch.Tensor], a: torch.Tensor,
                b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor, hk: int, hv: int, d: int, *,
                cu_seqlens: torch.Tensor, eps: float = 1e-6, out_dtype: Optional[torch.dtype] = None):
    """Packed tokens: z [N, C] (C = (2 hk + hv) d, bf16 or fp32, row stride free), conv_w [C, K], prefix
    [num_seqs, K - 1, C] or None, a, b [N, hv], A_log, dt_bias [hv], cu_seqlens [num_seqs + 1]. Returns q, k, v
    [N, hv, d] in ``out_dtype`` (default z's dtype), g, beta [N, hv] fp32 (``hibrit.py:163-177``)."""
    dev = require_device(z, conv_w, prefix, a, b, A_log, dt_bias, cu_seqlens)
    require_no_grad(z, conv_w, prefix, a, b)
    N, C = z.shape
    if C != (2 * hk + hv) * d or z.stride(1) != 1:
        raise BifrostError(f"z must be [N, {(2 * hk + hv) * d}] with unit channel stride, got {tuple(z.shape)}")
    K = conv_w.shape[-1]
    num_seqs = cu_seqlens.numel() - 1
    if z.dtype not in (torch.float32, torch.bfloat16):
        raise BifrostError(f"z dtype {z.dtype} not supported")
    if prefix is not None:
        prefix = prefix.to(z.dtype).contiguous()
        if prefix.shape != (num_seqs, K - 1, C):
            raise BifrostError(f"prefix must be [{num_seqs}, {K - 1}, {C}], got {tuple(prefix.shape)}")
    odt = out_dtype or z.dtype
    w = conv_w.float().reshape(C, K).contiguous()
    a, b = a.float().reshape(N, hv).contiguous(), b.float().reshape(N, hv).contiguous()
    A_log, dt_bias = A_log.float().contiguous(), dt_bias.float().contiguous()
    cu = cu_seqlens.to(device=dev, dtype=torch.int32).contiguous()
    q = torch.empty(N, hv, d, dtype=odt, device=dev)
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    g = torch.empty(N, hv, dtype=torch.float32, device=dev)
    beta = torch.empty_like(g)
    check(_lib.load().bf_gdn_conv_inputs(
        z.data_ptr(), z.stride(0), prefix.data_ptr() if prefix is not None else None, dtype_code(z.dtype),
        w.data_ptr(), K, a.data_ptr(), b.data_ptr(), A_log.data_ptr(), dt_bias.data_ptr(), cu.data_ptr(), num_seqs,
        N, hk, hv, d, float(eps), float(d ** -0.5), q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(),
        beta.data_ptr(), dtype_code(odt), stream_ptr(dev)), "bf_gdn_conv_inputs")
    return q, k, v, g, beta


def _fused_norm(dtype: torch.dtype, d: int) -> bool:
    """A bf16 layer with head dim <= 128 runs the GatedNorm inside the delta rule's output scan (bf_gdn_fwd_gated)."""
    return dtype == torch.bfloat16 and d <= 128


def gated_norm(o: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """weight * RMSNorm(o) * SiLU(z) over the last dim (``GatedNorm``, ``hibrit.py:118-129``). The result has z's
    dtype (the layer's dtype); a bf16 layer rounds where the reference does."""
    dev = require_device(o, z, weight)
    require_no_grad(o, z)
    d = o.shape[-1]
    if z.shape[-1] != d or z.numel() != o.numel():
        raise BifrostError("o and z must have the same shape")
    if z.dtype not in (torch.float32, torch.bfloat16):
        raise BifrostError(f"dtype {z.dtype} not supported")
    oc = o.contiguous() if o.dtype in (torch.float32, torch.bfloat16) else o.float().contiguous()
    zc = z.contiguous()
    w = weight.float().contiguous()
    out = torch.empty(z.shape, dtype=z.dtype, device=dev)
    check(_lib.load().bf_gated_norm(oc.data_ptr(), dtype_code(oc.dtype), zc.data_ptr(), w.data_ptr(),
                                    oc.numel() // d, d, float(eps), out.data_ptr(), dtype_code(z.dtype),
                                    stream_ptr(dev)), "bf_gated_norm")
    return out


class GatedNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x, z):
        return gated_norm(x, z, self.weight, self.eps)


class _Conv(nn.Module):
    def __init__(self, c: int, k: int) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(c, 1, k))


class GatedDeltaNet(nn.Module):
    """Drop-in for ``hibrit.GatedDeltaNet`` (``hibrit.py:136-184``), forward only."""

    def __init__(self, c: GdnLayerConfig) -> None:
        super().__init__()
        if c.lin_dk != c.lin_dv:
            raise BifrostError("the kernels need lin_dk == lin_dv")
        self.c = c
        self.kd, self.vd = c.lin_hk * c.lin_dk, c.lin_hv * c.lin_dv
        self.in_proj_qkv = nn.Linear(c.d, 2 * self.kd + self.vd, bias=False)
        self.in_proj_z = nn.Linear(c.d, self.vd, bias=False)
        self.in_proj_b = nn.Linear(c.d, c.lin_hv, bias=False)
        self.in_proj_a = nn.Linear(c.d, c.lin_hv, bias=False)
        self.conv1d = _Conv(2 * self.kd + self.vd, c.conv_k)
        self.dt_bias = nn.Parameter(torch.ones(c.lin_hv))
        self.A_log = nn.Parameter(torch.zeros(c.lin_hv))
        self.norm = GatedNorm(c.lin_dv, c.eps)
        self.out_proj = nn.Linear(self.vd, c.d, bias=False)

    @torch.no_grad()
    def forward(self, x, cache: Optional[dict] = None, start: int = 0):
        c, (b, t, _) = self.c, x.shape
        k1 = c.conv_k - 1
        z = self.in_proj_qkv(x)
        prefix = None if cache is None else cache.get("conv")
        s0 = None if cache is None else cache.get("S")
        step = s0 is not None and t == 1
        a, bb = self.in_proj_a(x), self.in_proj_b(x)
        q, k, v, g, beta = conv_inputs(z.reshape(b * t, -1), self.conv1d.weight[:, 0], prefix, a, bb, self.A_log,
                                       self.dt_bias, c.lin_hk, c.lin_hv, c.lin_dk,
                                       cu_seqlens=_seqlens(b, t, x.device),
                                       out_dtype=torch.float32 if step else None)
        if cache is not None:
            full = z if prefix is None else torch.cat((prefix.to(z.dtype), z), 1)
            cache["conv"] = F.pad(full, (0, 0, max(0, k1 - full.size(1)), 0))[:, -k1:]
        zg = self.in_proj_z(x).view(b, t, c.lin_hv, c.lin_dv)
        fused = not step and _fused_norm(q.dtype, c.lin_dv)
        if step:
            o, s = gdn_step(q, k, v, g, beta, s0)
            o = o.to(x.dtype)
        elif fused:                       # the output scan applies the GatedNorm to its rows (same bits)
            o, s = gdn_forward(q, k, v, g, beta, num_seqs=b, initial_state=s0,
                               gated_norm=(zg, self.norm.weight, self.norm.eps))
        else:
            o, s = gdn_forward(q, k, v, g, beta, num_seqs=b, initial_state=s0, out_dtype=x.dtype)
        if cache is not None:
            cache["S"] = s
        if not fused:
            o = self.norm(o.view(b, t, c.lin_hv, c.lin_dv), zg)
        return self.out_proj(o.reshape(b, t, self.vd))


@torch.no_grad()
def gdn_layer_packed(m: GatedDeltaNet, z: torch.Tensor, a: torch.Tensor, b: torch.Tensor, zg: torch.Tensor,
                     cu_seqlens: torch.Tensor, prefix: Optional[torch.Tensor] = None,
                     initial_state: Optional[torch.Tensor] = None, segment_chunks: int = 0):
    """The layer core between the projections on packed variable-length sequences: z [N, C], a, b [N, hv],
    zg [N, hv * d] (the in_proj_z output), cu_seqlens [num_seqs + 1]. Returns (gated-norm output [N, hv * d] in z's
    dtype, final state [num_seqs, hv, d, d] fp32); the new conv caches are the last K - 1 rows of each sequence."""
    c = m.c
    num_seqs = cu_seqlens.numel() - 1
    q, k, v, g, beta = conv_inputs(z, m.conv1d.weight[:, 0], prefix, a, b, m.A_log, m.dt_bias, c.lin_hk, c.lin_hv,
                                   c.lin_dk, cu_seqlens=cu_seqlens, eps=1e-6)
    if _fused_norm(q.dtype, c.lin_dv):
        out, s = gdn_forward(q, k, v, g, beta, num_seqs=num_seqs, cu_seqlens=cu_seqlens, initial_state=initial_state,
                             segment_chunks=segment_chunks, gated_norm=(zg.view(q.shape), m.norm.weight, m.norm.eps))
    else:
        o, s = gdn_forward(q, k, v, g, beta, num_seqs=num_seqs, cu_seqlens=cu_seqlens, initial_state=initial_state,
                           out_dtype=z.dtype, segment_chunks=segment_chunks)
        out = gated_norm(o, zg.view(o.shape), m.norm.weight, m.norm.eps)
    return out.view(z.shape[0], c.lin_hv * c.lin_dv), s
