"""ctypes binding of ``libtace_hip.so`` (the C ABI in ``include/tace_hip.h``).

The library is loaded from the package tree (``tace_amd/_lib``).  There is no
fallback: if it is missing or cannot be loaded, every operator raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libtace_hip.so")

F32, F64 = 0, 1

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()

_c_int, _c_i32, _c_i64, _c_dbl = ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_double
_vp, _cp = ctypes.c_void_p, ctypes.c_char_p

_SIGS = {
    "tace_last_error": (_cp, []),
    "tace_abi_version": (_c_int, []),
    "tace_mark_phase_event": (_c_int, [_vp]),
    "tace_tp_num_variants": (_c_int, []),
    "tace_tp_variant_key": (_cp, [_c_int]),
    "tace_tp_find": (_c_int, [_cp]),
    "tace_tp_dims": (_c_int, [_c_int, _vp, _vp, _vp, _vp]),
    "tace_edge_tp_workspace_elems": (_c_i64, [_c_int, _c_i64, _c_i32, _c_i32]),
    "tace_edge_tp_fwd": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32,
                                  _c_i32, _vp, _vp]),
    "tace_edge_tp_bwd": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32,
                                  _c_i32, _vp, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp]),
    "tace_edge_tp_fwd_rows": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64,
                                       _c_i32, _c_i32, _vp, _vp]),
    "tace_edge_tp_bwd_rows": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64,
                                       _c_i32, _c_i32, _vp, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp]),
    "tace_edge_pairs": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _vp]),
    "tace_radial_mlp_out_bwd_pairs_f32": (_c_int, [_vp, _vp, _vp, _c_i64, _c_i32, ctypes.c_float, _vp, _vp, _vp]),
    "tace_edge_tp_bwd_noalloc": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64,
                                          _c_i32, _c_i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tace_edge_rtp_fwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _c_i64, _c_i64,
                                   _c_i32, _c_i32, _vp, _vp, _vp]),
    "tace_edge_rtp_workspace_elems": (_c_i64, [_c_int, _c_i64, _c_i32, _c_i32]),
    "tace_edge_rtp_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _c_i64,
                                   _c_i64, _c_i32, _c_i32, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp]),
    "tace_edge_vec_fwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp]),
    "tace_edge_vec_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp]),
    "tace_uuu_fwd": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _vp, _vp]),
    "tace_uuu_workspace_elems": (_c_i64, [_c_int, _c_i64, _c_i32, _c_i32]),
    "tace_uuu_bwd": (_c_int, [_c_int, _c_int, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _vp, _vp, _vp, _vp, _c_i64,
                              _c_i32, _vp]),
    "tace_edge_basis_fwd": (_c_int, [_c_int, _vp, _c_i64, _c_i32, _vp, _c_dbl, _c_dbl, _c_i32, _c_i32, _vp, _vp, _vp]),
    "tace_edge_basis_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _c_i64, _c_i32, _vp, _c_dbl, _c_dbl, _c_i32, _c_i32,
                                     _vp, _vp]),
    "tace_edge_wigner_fwd": (_c_int, [_c_int, _vp, _c_i64, _c_i32, _vp, _vp]),
    "tace_edge_wigner_bwd": (_c_int, [_c_int, _vp, _vp, _c_i64, _c_i32, _vp, _vp]),
    "tace_tece_score_fwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _vp, _vp]),
    "tace_tece_score_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _c_i32, _vp, _vp,
                                     _vp, _vp]),
    "tace_graph_softmax_fwd": (_c_int, [_c_int, _vp, _vp, _vp, _c_i64, _c_i32, _vp, _vp]),
    "tace_graph_softmax_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _vp, _vp]),
    "tace_tece_rotate_out_fwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32,
                                          _c_i32, _vp, _vp]),
    "tace_tece_rotate_out_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32,
                                          _c_i32, _vp, _vp, _vp, _vp]),
    "tace_edge_rotate_in_fwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32, _vp, _vp,
                                         _vp, _vp]),
    "tace_edge_rotate_in_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32,
                                         _c_i32, _vp, _vp, _vp, _vp, _c_i32, _vp]),
    "tace_edge_rotate_in_bwd_runs": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64,
                                              _c_i32, _c_i32, _vp, _vp, _vp, _vp, _c_i32, _vp]),
    "tace_tece_edge_ace_fwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32, _vp, _vp, _vp, _vp,
                                        _vp]),
    "tace_tece_edge_ace_bwd": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_i32,
                                        _vp, _vp, _vp, _vp, _vp]),
    "tace_radial_mlp_fwd": (_c_int, [_c_int, _vp, _c_i64, _c_i32, _c_i32, _vp, _vp, _vp]),
    "tace_radial_mlp_bwd": (_c_int, [_c_int, _vp, _vp, _c_i64, _c_i32, _c_i32, _vp, _vp, _vp]),
    "tace_radial_mlp_out_f32": (_c_int, [_vp, _vp, _c_i64, _c_i32, ctypes.c_float, _vp, _vp]),
    "tace_radial_mlp_out_bwd_f32": (_c_int, [_vp, _vp, _c_i64, _c_i32, ctypes.c_float, _vp, _vp]),
    "tace_seg_linear": (_c_int, [_c_int, _c_i32, _c_i32, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _c_dbl, _vp]),
    "tace_bf16x3_split_blocks": (_c_int, [_vp, _vp, _vp, _c_i64, _vp, _c_i64, _vp]),
    "tace_seg_linear_presplit": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _c_i64, _vp, _c_dbl, _vp]),
    "tace_seg_linear_ks_rows": (_c_i32, [_c_i32]),
    "tace_so2_gemm_bf16": (_c_int, [_vp, _c_i64, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32, _vp]),
    "tace_so2_gemm_bf16_kt": (_c_int, [_vp, _c_i64, _vp, _vp, _vp, _c_i64, _c_i64, _c_i32, _c_i32, _vp]),
    "tace_seg_linear_presplit_ks": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i32, _c_dbl, _vp]),
    "tace_seg_linear_presplit_frag": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i32, _c_dbl, _vp]),
    "tace_seg_linear_presplit_frag_split": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i32, _c_i32, _vp,
                                                     _c_i64, _c_dbl, _vp]),
    "tace_nl_workspace_bytes": (_c_i64, [_c_i64, _vp, _vp, _c_dbl]),
    "tace_nl_count": (_c_int, [_vp, _c_i64, _vp, _vp, _c_dbl, _vp, _c_i64, _vp, _vp]),
    "tace_nl_fill": (_c_int, [_vp, _c_i64, _vp, _vp, _c_dbl, _vp, _vp, _vp, _vp, _vp]),
    "tace_nl_batch_plan": (_c_i64, [_c_i32, _vp, _vp, _vp, _c_dbl, _vp, _c_i64, _vp, _vp]),
    "tace_nl_batch_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "tace_nl_batch_count": (_c_int, [_vp, _c_i64, _c_i32, _vp, _c_i64, _vp, _c_i64, _c_i32, _vp, _vp]),
    "tace_nl_batch_fill": (_c_int, [_vp, _c_i64, _c_i32, _vp, _c_i64, _vp, _c_i64, _c_i32, _vp, _vp, _vp, _vp]),
    "tace_rows_accumulate": (_c_int, [_c_int, _vp, _c_i64, _c_i64, _vp, _vp, _vp, _c_i64, _vp, _c_i64, _vp]),
    "tace_graph_sum": (_c_int, [_c_int, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    "tace_narrow_linear": (_c_int, [_c_int, _vp, _c_i64, _c_i32, _vp, _vp, _c_i32, _vp, _vp]),
    "tace_rows_accumulate_runs": (_c_int, [_c_int, _vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_i32, _vp, _c_i64,
                                           _vp]),
    "tace_scan_i32": (_c_int, [_vp, _c_i64, _vp, _vp]),
}

EXPORTED = tuple(_SIGS)


class NativeError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the library once (raises if it is absent -- no CPU fallback)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise NativeError(
                        f"libtace_hip.so not found at {LIB_PATH}; build it with "
                        "`python -m tace_amd.build` (hipcc, gfx950)")
                L = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in _SIGS.items():
                    f = getattr(L, name)
                    f.restype = res
                    f.argtypes = args
                _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().tace_last_error()
        raise NativeError(f"{what or 'tace_hip'} failed ({rc}): {msg.decode() if msg else ''}")


def dtype_code(dtype) -> int:
    import torch

    if dtype == torch.float32:
        return F32
    if dtype == torch.float64:
        return F64
    raise NativeError(f"unsupported dtype {dtype}; TACE HIP kernels take float32 or float64")


def ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_ptr(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream
