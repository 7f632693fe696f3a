"""Device-side plumbing shared by the operator wrappers: dtype codes, workspace, stream, the GDN launcher."""
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import BifrostError, check

SUPPORTED_D = (64, 128, 256)


def require_device(*tensors) -> torch.device:
    """All tensors must live on one HIP device: the operators have no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise BifrostError("heimdall_amd operators run on the GPU only (got a tensor on "
                               f"{t.device}); use the reference implementation for CPU tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise BifrostError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise BifrostError("no tensor argument")
    return dev


def require_no_grad(*tensors) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise BifrostError("heimdall_amd kernels are forward-only; call under torch.no_grad() or detach the inputs")


def compute_dtype(*tensors) -> torch.dtype:
    """Operand dtype of the kernels: bf16 (bf16 MFMA operands, fp32 accumulation) when every input is bf16, else fp32.
    fp16 inputs are widened to fp32, never rounded to bf16 (the reference computes in fp32 with autocast off,
    ``kernels.py:101``, ``hibrit.py:336-339``)."""
    for t in tensors:
        if t.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise BifrostError(f"unsupported input dtype {t.dtype}")
    return torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in tensors) else torch.float32


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dt == torch.float32:
        return _lib.DTYPE_F32
    raise BifrostError(f"unsupported dtype {dt}")


def stream_ptr(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def gdn_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor, *,
                num_seqs: int, cu_seqlens: Optional[torch.Tensor] = None, initial_state: Optional[torch.Tensor] = None,
                scale: float = 1.0, out_dtype: torch.dtype = torch.float32, phases: int = _lib.PHASE_ALL,
                out: Optional[torch.Tensor] = None, final_state: Optional[torch.Tensor] = None,
                ws: Optional[torch.Tensor] = None, segment_chunks: int = 0,
                gated_norm: Optional[Tuple[torch.Tensor, torch.Tensor, float]] = None):
    """Packed GQA gated delta rule on the GPU.

    q [N, G*R, D], k [N, G, D], v [N, G, D], g/beta [N, G]; cu_seqlens int32 [num_seqs + 1] on the device or None
    (equal sequences). ``segment_chunks``: 64-token chunks per independently scanned segment (0 = chosen from the
    problem size). Returns (o [N, G*R, D] out_dtype, final_state [num_seqs, G, D, D] fp32).

    ``gated_norm`` = (z [N, G*R, D] bf16, w [D], eps): bf16 inputs, D <= 128; the output rows go through the
    native layer's GatedNorm inside the output scan (``bf_gdn_fwd_gated``), the same bits as ``gated_norm`` applied
    to the bf16 output, and the bf16 result is returned in place of o.
    """
    dev = require_device(q, k, v, g, beta, cu_seqlens, initial_state)
    N, H, D = q.shape
    G = k.shape[1]
    if H % G or k.shape != (N, G, D) or v.shape != (N, G, D) or g.shape != (N, G) or beta.shape != (N, G):
        raise BifrostError(f"inconsistent shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} "
                           f"g{tuple(g.shape)} beta{tuple(beta.shape)}")
    if D not in SUPPORTED_D:
        raise BifrostError(f"head dim {D} not supported (supported: {SUPPORTED_D})")
    R = H // G
    cdt = compute_dtype(q, k, v)
    q, k, v = (t.to(cdt).contiguous() for t in (q, k, v))
    g, beta = g.float().contiguous(), beta.float().contiguous()
    if cu_seqlens is not None:
        cu_seqlens = cu_seqlens.to(device=dev, dtype=torch.int32).contiguous()
        if cu_seqlens.numel() != num_seqs + 1:
            raise BifrostError("cu_seqlens must hold num_seqs + 1 offsets")
    elif N % num_seqs:
        raise BifrostError("token count is not a multiple of num_seqs")
    s0 = None
    if initial_state is not None:
        s0 = initial_state.float().contiguous()
        if s0.shape != (num_seqs, G, D, D):
            raise BifrostError(f"initial_state must be [{num_seqs}, {G}, {D}, {D}], got {tuple(s0.shape)}")
    lib = _lib.load()
    nbytes = _lib.ctypes.c_size_t(0)
    check(lib.bf_gdn_workspace_size(N, num_seqs, G, R, D, dtype_code(cdt), int(segment_chunks),
                                    _lib.ctypes.byref(nbytes)), "bf_gdn_workspace_size")
    if ws is None or ws.numel() < nbytes.value:
        ws = workspace(nbytes.value, dev)
    if gated_norm is not None:
        gz, gw, geps = gated_norm
        if cdt != torch.bfloat16 or D > 128 or gz.dtype != torch.bfloat16 or gz.numel() != N * H * D:
            raise BifrostError("the fused GatedNorm takes bf16 inputs and z rows [N, H, D] with D <= 128")
        gz = gz.reshape(N, H, D).contiguous()
        gw = gw.detach().float().contiguous()
        if gw.numel() != D or (out is not None and out.dtype != torch.bfloat16):
            raise BifrostError("the fused GatedNorm takes w [D] and writes a bf16 output")
        out_dtype = torch.bfloat16
    o = out if out is not None else torch.empty(N, H, D, dtype=out_dtype, device=dev)
    s_out = final_state if final_state is not None else torch.empty(num_seqs, G, D, D, dtype=torch.float32,
                                                                     device=dev)
    if gated_norm is not None:
        check(lib.bf_gdn_fwd_gated(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                                   cu_seqlens.data_ptr() if cu_seqlens is not None else None, num_seqs, N, G, R, D,
                                   float(scale), s0.data_ptr() if s0 is not None else None, gz.data_ptr(),
                                   gw.data_ptr(), float(geps), o.data_ptr(), s_out.data_ptr(), int(segment_chunks),
                                   ws.data_ptr(), ws.numel(), phases, stream_ptr(dev)),
              "bf_gdn_fwd_gated")
        return o, s_out
    check(lib.bf_gdn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                         cu_seqlens.data_ptr() if cu_seqlens is not None else None, num_seqs, N, G, R, D,
                         dtype_code(cdt), float(scale), s0.data_ptr() if s0 is not None else None, o.data_ptr(),
                         dtype_code(o.dtype), s_out.data_ptr(), int(segment_chunks), ws.data_ptr(), ws.numel(), phases,
                         stream_ptr(dev)),
          "bf_gdn_fwd")
    return o, s_out
