"""Attention of the kept full-attention layers (the teacher) over a KV cache, with Quest-style retrieval, on the GPU.

Drop-in for ``HybridAttention._teacher`` and ``set_retrieval`` (``Heimdall/heimdall/hibrit.py:275-299``), with the
reference's cache contract: ``cache["k"]`` / ``cache["v"]`` hold the keys (RoPE applied) and values [B, G, n, D] of
every position so far. Here they are views of capacity buffers (``cache["k_buf"]`` / ``cache["v_buf"]`` [B, G, cap, D],
grown by half again when full), so a decode step writes one row instead of concatenating the whole cache again; a
cache filled elsewhere (plain tensors under "k" / "v") is adopted on the next call.

The attended keys are the reference's on every path:
  retrieval (t == 1, or any t when ``prefill`` is set, once n - sinks - window >= k * block):
      ``bf_kv_block_summary`` on the full blocks not yet summarised (min / max kept in the cache), ``bf_kv_select``,
      ``bf_kv_attention`` over the sinks, the selected blocks and the window;
  t <= 16 without retrieval: ``bf_kv_attention`` (split-K over the cache, each query up to its own position);
  t == n: ``bf_window_fwd`` with a window as long as the sequence (causal, MFMA);
  t < n:  ``bf_window_fwd`` with the cache buffer as its ring, so every earlier position is visible.
"""
from typing import Optional

import ctypes
import torch

from . import _lib
from ._device import BifrostError, check, dtype_code, require_device, require_no_grad, stream_ptr, workspace
from .motor import blockwise_attention

SMALL_T = 16                 # queries per sequence up to which the split-K kernel serves plain (causal) attention
WS_BUDGET = 1 << 30          # workspace bytes per bf_kv_attention call (longer query runs are chunked)


def set_retrieval(self, k: Optional[int] = 16, block: int = 64, window: int = 2048, sinks: int = 4,
                  prefill: bool = False):
    """Retrieval attention for a full-attention layer (``hibrit.py:292-299``): each query attends exactly to the sinks,
    the recent window (from the block boundary at or before pos - window + 1) and the k key blocks with the highest
    upper bound on q.k per KV head. prefill=False applies it to single-token decode only; k=0 keeps the sinks and
    the window; k=None turns it off."""
    if k is not None and (k < 0 or k > _lib.KV_MAX_K or block <= 0 or window <= 0 or sinks < 0):
        raise BifrostError(f"retrieval needs 0 <= k <= {_lib.KV_MAX_K}, block > 0, window > 0, sinks >= 0")
    self.retrieval = None if k is None else dict(k=k, block=block, window=window, sinks=sinks, prefill=prefill)


def uses_retrieval(ret: Optional[dict], t: int, n: int) -> bool:
    """The reference's condition (``hibrit.py:281``)."""
    return ret is not None and (t == 1 or bool(ret.get("prefill"))) and \
        n - ret["sinks"] - ret["window"] >= ret["k"] * ret["block"]


def _kv_view(t: torch.Tensor):
    """(tensor, per-(b, g) stride, per-position stride) of a [B, G, n, D] key or value tensor as the kernels address
    it: row (b, g, p) at (b * G + g) * s_bg + p * s_p."""
    G = t.shape[1]
    if (t.stride(-1) != 1 or t.stride(0) != G * t.stride(1) or t.stride(1) % 8 or t.stride(2) % 8
            or t.data_ptr() % 16):
        t = t.contiguous()
    return t, t.stride(1), t.stride(2)


def summary_buffers(B: int, G: int, D: int, nb_cap: int, dtype: torch.dtype, dev):
    """Empty block summaries (kmin, kmax) in the keys' dtype and the kernels' layout [B, G, D / GS, nb_cap, GS],
    GS = 16 bytes / element (a block's min / max of a key dimension is one of the key values: no rounding)."""
    gs = 16 // torch.empty(0, dtype=dtype).element_size()
    kmin = torch.empty(B, G, D // gs, nb_cap, gs, dtype=dtype, device=dev)
    return kmin, torch.empty_like(kmin)


def summaries_as_blocks(s: torch.Tensor) -> torch.Tensor:
    """[B, G, D / GS, nb_cap, GS] -> [B, G, nb_cap, D] (a copy for inspection)."""
    B, G, C, nb, gs = s.shape
    return s.permute(0, 1, 3, 2, 4).reshape(B, G, nb, gs * C)


def kv_block_summary(k: torch.Tensor, sinks: int, block: int, first_block: int, nb: int, kmin: torch.Tensor,
                     kmax: torch.Tensor) -> None:
    """kmin / kmax (``summary_buffers``; written in place) <- the per-dimension key minimum and maximum of the blocks
    first_block .. nb - 1 of k [B, G, n, D] (block j = keys sinks + j block ..)."""
    dev = require_device(k, kmin, kmax)
    k, s_bg, s_p = _kv_view(k)
    B, G, _, D = k.shape
    check(_lib.load().bf_kv_block_summary(k.data_ptr(), dtype_code(k.dtype), B, G, D, s_bg, s_p, sinks, block,
                                          first_block, nb, kmin.shape[3], kmin.data_ptr(), kmax.data_ptr(),
                                          stream_ptr(dev)), "bf_kv_block_summary")


def kv_select(q: torch.Tensor, n: int, ret: dict, kmin: torch.Tensor, kmax: torch.Tensor) -> torch.Tensor:
    """q [B, T, H, D] (the queries at positions n - T .. n - 1), summaries from ``kv_block_summary`` -> the selected block ids
    [B, T, G, k] int32 (-1 past the candidates)."""
    dev = require_device(q, kmin, kmax)
    B, T, H, D = q.shape
    G = kmin.shape[1]
    q = q.contiguous()
    sel = torch.empty(B, T, G, max(ret["k"], 1), dtype=torch.int32, device=dev)
    check(_lib.load().bf_kv_select(q.data_ptr(), dtype_code(q.dtype), B, T, G, H // G, D, n, ret["sinks"],
                                   ret["window"], ret["block"], kmin.data_ptr(), kmax.data_ptr(), kmin.shape[3],
                                   ret["k"], sel.data_ptr(), stream_ptr(dev)), "bf_kv_select")
    return sel


def kv_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, n: int, ret: Optional[dict] = None,
                 sel: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.float32,
                 scale: Optional[float] = None) -> torch.Tensor:
    """q [B, T, H, D] at positions n - T .. n - 1 over the first n rows of k / v [B, G, >= n, D] (one dtype, bf16 or
    fp32). Without ``ret`` each query attends to every key up to its position; with ``ret`` to the sinks, the blocks
    of ``sel`` and the window. Returns o [B, T, H, D] in ``out_dtype``."""
    dev = require_device(q, k, v, sel)
    B, T, H, D = q.shape
    G = k.shape[1]
    if H % G or k.shape[0] != B or v.shape[:2] != k.shape[:2] or k.shape[-1] != D or v.shape[-1] != D:
        raise BifrostError(f"inconsistent shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if k.shape[2] < n or v.shape[2] < n or T > n:
        raise BifrostError(f"{T} queries over {n} keys need n >= T rows in k and v")
    if not (q.dtype == k.dtype == v.dtype):
        raise BifrostError(f"q, k, v dtypes differ: {q.dtype}, {k.dtype}, {v.dtype}")
    q = q.contiguous()
    k, k_bg, k_p = _kv_view(k)
    v, v_bg, v_p = _kv_view(v)
    lib = _lib.load()
    on = ret is not None
    S, W, L, K = (ret["sinks"], ret["window"], ret["block"], ret["k"]) if on else (0, 0, 1, 0)
    if on and K > 0 and (sel is None or sel.shape != (B, T, G, K) or sel.dtype != torch.int32):
        raise BifrostError("retrieval with k > 0 needs sel [B, T, G, k] int32 from kv_select")
    sel_p = sel.contiguous().data_ptr() if on and K > 0 else None
    o = torch.empty(B, T, H, D, dtype=out_dtype, device=dev)
    nbytes = ctypes.c_size_t(0)
    check(lib.bf_kv_attention_workspace_size(B, T, G, H // G, D, n, int(on), S, W, L, K, ctypes.byref(nbytes)),
          "bf_kv_attention_workspace_size")
    ws = workspace(nbytes.value, dev)
    check(lib.bf_kv_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), dtype_code(q.dtype), B, T, G, H // G, D, n,
                              k_bg, k_p, v_bg, v_p, int(on), S, W, L, sel_p, K,
                              float(D ** -0.5 if scale is None else scale), ws.data_ptr(), nbytes.value, o.data_ptr(),
                              dtype_code(out_dtype), stream_ptr(dev)), "bf_kv_attention")
    return o


def _appendable(x: torch.Tensor) -> bool:
    """Rows the append kernel reads directly: D contiguous, 16-byte aligned, strides in whole 16-byte vectors."""
    return x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in x.stride()[:3])


def _append(cache: dict, kr: torch.Tensor, vt: torch.Tensor):
    """Appends the new rows kr / vt [B, G, t, D] to the cache's capacity buffers; cache["k"] / cache["v"] become
    [B, G, n, D] views of them. Returns (k_buf, v_buf, n, adopted) — adopted: the history came from plain tensors."""
    B, G, t, D = kr.shape
    kb, vb = cache.get("k_buf"), cache.get("v_buf")
    k_old, v_old = cache.get("k"), cache.get("v")
    n0 = 0 if k_old is None else k_old.shape[2]
    own = (kb is not None and k_old is not None and k_old.data_ptr() == kb.data_ptr() and
           v_old.data_ptr() == vb.data_ptr() and k_old.shape[2] <= kb.shape[2] and kb.dtype == kr.dtype and
           kb.shape[:2] == (B, G) and kb.shape[3] == D)
    adopted = k_old is not None and not own
    n = n0 + t
    if not own or kb.shape[2] < n:
        cap = max(256, -(-(n + n // 2) // 256) * 256)
        nk = torch.empty(B, G, cap, D, dtype=kr.dtype, device=kr.device)
        nv = torch.empty(B, G, cap, D, dtype=vt.dtype, device=vt.device)
        if n0:
            nk[:, :, :n0] = k_old
            nv[:, :, :n0] = v_old
        kb, vb = nk, nv
        cache["k_buf"], cache["v_buf"] = kb, vb
        cache.pop("ring_pos", None)
    kr = kr if _appendable(kr) else kr.contiguous()
    vt = vt if _appendable(vt) else vt.contiguous()
    check(_lib.load().bf_kv_append(kr.data_ptr(), kr.stride(0), kr.stride(1), kr.stride(2), vt.data_ptr(),
                                   vt.stride(0), vt.stride(1), vt.stride(2), dtype_code(kb.dtype), B, G, t, D,
                                   kb.data_ptr(), vb.data_ptr(), kb.shape[2], n0, stream_ptr(kr.device)),
          "bf_kv_append")
    cache["k"], cache["v"] = kb[:, :, :n], vb[:, :, :n]
    return kb, vb, n, adopted


def _summaries(cache: Optional[dict], k: torch.Tensor, n: int, ret: dict, fresh: bool):
    """Block min / max of the full blocks of k's first n rows (``summary_buffers`` layout); kept in the cache
    ("kv_kmin", "kv_kmax", "kv_sum") so each call summarises only blocks completed since the last one."""
    B, G, cap, D = k.shape
    S, L = ret["sinks"], ret["block"]
    nb = max(0, (n - S) // L)
    meta = None if cache is None or fresh else cache.get("kv_sum")
    if meta is not None and (meta["S"] != S or meta["L"] != L or cache["kv_kmin"].dtype != k.dtype or
                             cache["kv_kmin"].shape[:2] != (B, G)):
        meta = None
    done = 0 if meta is None else min(meta["nb"], nb)
    if meta is not None and meta["nb_cap"] >= nb:
        kmin, kmax = cache["kv_kmin"], cache["kv_kmax"]
    else:
        kmin, kmax = summary_buffers(B, G, D, max(1, (max(cap, n) - S) // L + 1), k.dtype, k.device)
        if done:                                        # grown cache: keep the finished blocks
            kmin[:, :, :, :done] = cache["kv_kmin"][:, :, :, :done]
            kmax[:, :, :, :done] = cache["kv_kmax"][:, :, :, :done]
    if nb > done:
        kv_block_summary(k, S, L, done, nb, kmin, kmax)
    if cache is not None:
        cache["kv_kmin"], cache["kv_kmax"] = kmin, kmax
        cache["kv_sum"] = dict(S=S, L=L, nb=nb, nb_cap=kmin.shape[3])
    return kmin, kmax


def _trailing_queries(q, k, v, n, t, ret, kmin, kmax, out_dtype):
    """kv_attention for the t queries at positions n - t .. n - 1, in runs of queries whose workspace fits the budget
    (a run ending at position e is the last e keys' query block: each query sees only keys up to itself)."""
    B, _, H, D = q.shape
    max_keys = n if ret is None else min(n, ret["sinks"] + ret["k"] * ret["block"] + ret["window"] + ret["block"] - 1)
    per_q = 4 * B * H * (D + 2) * -(-max_keys // 512)            # workspace bytes per query (512-key splits)
    run = max(1, min(t, WS_BUDGET // per_q))
    if ret is not None:
        run = max(run, ret["sinks"])          # every run ends at or past the sinks (positions the sinks occupy)
    if run >= t:
        sel = kv_select(q, n, ret, kmin, kmax) if ret is not None and ret["k"] > 0 else None
        return kv_attention(q, k, v, n, ret, sel, out_dtype)
    o = torch.empty(B, t, H, D, dtype=out_dtype, device=q.device)
    for i0 in range(0, t, run):
        i1 = min(t, i0 + run)
        e = n - t + i1
        qc = q[:, i0:i1].contiguous()
        sel = kv_select(qc, e, ret, kmin, kmax) if ret is not None and ret["k"] > 0 else None
        o[:, i0:i1] = kv_attention(qc, k, v, e, ret, sel, out_dtype)
    return o


def _prefix_attention(qr, kb, vb, n, cache, out_dtype):
    """The t queries at positions n - t .. n - 1 over every earlier key: the window kernel with the cache buffer as a
    ring of W = capacity slots (slot p = position p) and the last t rows as the chunk."""
    dev = qr.device
    B, H, t, D = qr.shape
    G, cap = kb.shape[1], kb.shape[2]
    rp = cache.get("ring_pos")
    if rp is None or rp.numel() != cap:
        rp = torch.arange(cap, dtype=torch.int64, device=dev)
        cache["ring_pos"] = rp
    q = qr if qr.stride(-1) == 1 else qr.contiguous()
    kc, vc = kb[:, :, n - t:n], vb[:, :, n - t:n]
    o = torch.empty(B, t, H, D, dtype=out_dtype, device=dev)
    st = lambda x: (int(x.stride(0)), int(x.stride(1)), int(x.stride(2)))
    check(_lib.load().bf_window_fwd(B, G, H // G, D, t, cap, 0, n - t, dtype_code(kb.dtype), q.data_ptr(), *st(q),
                                    kc.data_ptr(), *st(kc), vc.data_ptr(), *st(vc), kb.data_ptr(), vb.data_ptr(),
                                    rp.data_ptr(), None, None, 0, 0, None, 0, None, None, None, o.data_ptr(),
                                    dtype_code(out_dtype), None, stream_ptr(dev)), "bf_window_fwd")
    return o


@torch.no_grad()
def teacher(self, qr: torch.Tensor, kr: torch.Tensor, v: torch.Tensor, cache: Optional[dict]):
    """``_teacher(qr, kr, v, cache)`` (``hibrit.py:275-290``): qr [B, H, t, D], kr [B, G, t, D] (RoPE applied),
    v [B, t, G, D]. Returns o [B, t, H, D] in qr's dtype."""
    dev = require_device(qr, kr, v)
    require_no_grad(qr, kr, v)
    B, H, t, D = qr.shape
    G = kr.shape[1]
    if H % G or kr.shape != (B, G, t, D) or v.shape != (B, t, G, D):
        raise BifrostError(f"inconsistent shapes qr{tuple(qr.shape)} kr{tuple(kr.shape)} v{tuple(v.shape)}")
    cdt = torch.bfloat16 if qr.dtype == kr.dtype == v.dtype == torch.bfloat16 else torch.float32
    kr, vt = kr.to(cdt), v.to(cdt).transpose(1, 2)
    if cache is not None:
        if "k" in cache and cache["k"].dtype != cdt:
            cache["k"], cache["v"] = cache["k"].to(cdt), cache["v"].to(cdt)
        kb, vb, n, adopted = _append(cache, kr, vt)
        k_all, v_all = cache["k"], cache["v"]
    else:
        kb = vb = None
        n, adopted = t, False
        k_all, v_all = kr, vt
    ret = getattr(self, "retrieval", None)
    use_ret = uses_retrieval(ret, t, n)
    if use_ret or t <= SMALL_T:
        q = qr.to(cdt).transpose(1, 2).contiguous()
        kmin = kmax = None
        if use_ret and ret["k"] > 0:
            kmin, kmax = _summaries(cache, kb if kb is not None else k_all, n, ret, adopted)
        src_k = kb if kb is not None else k_all
        src_v = vb if vb is not None else v_all
        o = _trailing_queries(q, src_k, src_v, n, t, ret if use_ret else None, kmin, kmax, qr.dtype)
    elif t == n:
        o = blockwise_attention(qr.to(cdt), k_all, v_all)
    else:
        o = _prefix_attention(qr.to(cdt), kb, vb, n, cache, qr.dtype)
    return o.to(qr.dtype)
