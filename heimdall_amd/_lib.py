"""ctypes binding of ``libbifrost_hip.so`` (the C ABI declared in ``include/bifrost.h``).

There is no fallback: if the library is missing or does not load, every operator raises.
"""
import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libbifrost_hip.so"

DTYPE_F32, DTYPE_BF16 = 0, 1
PHASE_PREP, PHASE_SUMMARY, PHASE_OUTPUT, PHASE_COMBINE = 1, 2, 4, 8
PHASE_STATES, PHASE_ALL = PHASE_SUMMARY | PHASE_COMBINE, 15
KV_MAX_K, KV_MAX_BLOCKS = 64, 16384      # bf_kv_select limits

_c_int, _c_i64, _c_sz, _vp, _fp = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float

# name -> (restype, argtypes); every symbol declared in include/bifrost.h
SIGNATURES = {
    "bf_version": (_c_int, []),
    "bf_status_string": (ctypes.c_char_p, [_c_int]),
    "bf_gdn_segment_chunks": (_c_int, [_c_i64, _c_int, _c_int, _c_int, _c_int]),
    "bf_gdn_workspace_size": (_c_int, [_c_i64, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                       ctypes.POINTER(_c_sz)]),
    "bf_gdn_fwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int, _fp, _vp,
                            _vp, _c_int, _vp, _c_int, _vp, _c_sz, _c_int, _vp]),
    "bf_gdn_step": (_c_int, [_vp] * 8 + [_c_int] * 4 + [_vp]),
    "bf_decode_workspace_size": (_c_int, [_c_int] * 5 + [ctypes.POINTER(_c_sz)]),
    "bf_decode_fwd": (_c_int, [_c_int] * 6 + [_c_i64] + [_c_int] * 3 + [_vp] * 12 + [_c_int] + [_vp] * 10 + [_c_sz, _vp]),
    "bf_decode_fwd_batch": (_c_int, [_c_int] * 6 + [_vp, _c_int, _c_int, _c_int] + [_vp] * 22 + [_c_sz, _vp]),
    "bf_student_decode_workspace_size": (_c_int, [_c_int] * 6 + [ctypes.POINTER(_c_sz)]),
    "bf_student_decode": (_c_int, [_c_int] * 6 + [_c_i64, _vp, _c_int, _c_int] + [_vp] * 19 + [_c_int]
                          + [_vp] * 9 + [_c_sz, _vp]),
    "bf_decode_fwd_noalloc": (_c_int, [_c_int] * 6 + [_c_i64] + [_c_int] * 3 + [_vp] * 12 + [_c_int] + [_vp] * 9 + [_vp]),
    "bf_window_fwd": (_c_int, [_c_int] * 7 + [_c_i64, _c_int] + ([_vp] + [_c_i64] * 3) * 3 + [_vp] * 5 + [_c_int] * 2
                      + [_vp, _c_int] + [_vp] * 4 + [_c_int, _vp, _vp]),
    "bf_mem_project": (_c_int, [_vp, _c_i64, _c_int, _c_int, _c_i64, _c_i64, _vp, _fp, _vp, _c_int, _c_int, _vp]),
    "bf_mem_gates": (_c_int, [_vp, _c_i64, _c_i64, _c_int, _c_i64, _vp, _vp, _vp, _c_i64, _c_int, _vp, _vp, _vp]),
    "bf_gate_project_workspace_size": (_c_int, [_c_i64, _c_int, _c_int, ctypes.POINTER(_c_sz)]),
    "bf_gate_project": (_c_int, [_vp, _c_i64, _c_int, _c_i64, _vp, _vp, _c_int, _vp, _vp, _vp, _c_int, _vp, _vp,
                                 _c_sz, _vp]),
    "bf_gdn_conv_inputs": (_c_int, [_vp, _c_i64, _vp, _c_int, _vp, _c_int] + [_vp] * 5 + [_c_int, _c_i64]
                           + [_c_int] * 3 + [_fp, _fp] + [_vp] * 5 + [_c_int, _vp]),
    "bf_gated_norm": (_c_int, [_vp, _c_int, _vp, _vp, _c_i64, _c_int, _fp, _vp, _c_int, _vp]),
    "bf_gdn_fwd_gated": (_c_int, [_vp] * 6 + [_c_int, _c_i64, _c_int, _c_int, _c_int, _fp, _vp, _vp, _vp, _fp, _vp, _vp,
                                       _c_int, _vp, _c_sz, _c_int, _vp]),
    "bf_gdn_bwd_workspace_size": (_c_int, [_c_int, _c_i64, _c_int, _c_int, _c_int, ctypes.POINTER(_c_sz)]),
    "bf_gdn_bwd": (_c_int, [_vp] * 6 + [_fp, _vp, _vp, _c_int, _c_i64, _c_int, _c_int, _c_int] + [_vp] * 7
                   + [_c_sz, _vp]),
    "bf_layer_prefill_workspace_size": (_c_int, [_c_int] * 6 + [ctypes.POINTER(_c_sz)]),
    "bf_layer_prefill_fwd": (_c_int, [_c_int] * 7 + [_c_i64, _c_int, _c_int] + ([_vp, _c_i64, _c_i64, _c_i64] * 3)
                             + [_vp, _c_int, _vp, _c_int] + [_vp] * 7 + [_c_int] + [_vp] * 7 + [_c_int]
                             + [_vp, _vp, _vp, _c_sz, _vp]),
    "bf_llama_state_floats": (_c_int, [_c_int] * 4 + [ctypes.POINTER(_c_i64)]),
    "bf_llama_state_pack": (_c_int, [_c_int] * 5 + [_c_i64, _c_int] + [_vp] * 8 + [_c_int, _vp, _vp, _vp]),
    "bf_llama_state_unpack": (_c_int, [_c_int] * 5 + [_c_i64, _c_int] + [_vp] * 9 + [_c_int, _vp, _vp]),
    "bf_kv_append": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64] + [_c_int] * 5
                     + [_vp, _vp, _c_i64, _c_i64, _vp]),
    "bf_kv_block_summary": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64] + [_c_int] * 5
                            + [_vp, _vp, _vp]),
    "bf_kv_select": (_c_int, [_vp] + [_c_int] * 6 + [_c_i64, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int, _vp,
                                                     _vp]),
    "bf_kv_attention_workspace_size": (_c_int, [_c_int] * 5 + [_c_i64] + [_c_int] * 5 + [ctypes.POINTER(_c_sz)]),
    "bf_kv_attention": (_c_int, [_vp, _vp, _vp] + [_c_int] * 6 + [_c_i64] * 5 + [_c_int] * 4
                        + [_vp, _c_int, _fp, _vp, _c_sz, _vp, _c_int, _vp]),
}

_LIB = None


class BifrostError(RuntimeError):
    pass


def load():
    """Load the library once; raise ``BifrostError`` if it is missing (build it with ``python -m heimdall_amd.build``)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise BifrostError(f"{LIB_PATH} not found: build it with `python -m heimdall_amd.build`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _LIB = lib
    return _LIB


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().bf_status_string(status).decode()
        raise BifrostError(f"{what} failed with status {status}: {msg}")
