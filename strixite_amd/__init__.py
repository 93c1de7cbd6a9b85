"""strixite_amd: strixite's MTP verify path on MI355X (gfx950), behind the C ABI of include/strixite_amd.h.

The compute is libstrixite_amd.so (hand-written HIP kernels, built by strixite_amd/build.py). This package only loads
it and passes device pointers: there is no CPU or PyTorch fallback - without the library every call raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libstrixite_amd.so")

SX_OK, SX_EINVAL, SX_EHIP, SX_EUNSUPPORTED = 0, 1, 2, 3
ACT_F32, ACT_BF16 = 0, 1
MOE_F32, MOE_WMMA_BF16, MOE_WMMA_F16 = 0, 1, 2


class SxError(RuntimeError):
    """A failed C-ABI call: status code + the library's message (the reference's strix::Error text)."""

    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class QView(ctypes.Structure):
    """sx_qview: Q4DeviceView / Q8DeviceView (runtime/q4_device.hpp:13-18, q8_device.hpp:12-17)."""
    _fields_ = [("q", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("minv", ctypes.c_void_p),
                ("N", ctypes.c_int64), ("K", ctypes.c_int64), ("G", ctypes.c_int64)]


class LogitCand(ctypes.Structure):
    """sx_logit_cand: LogitCand (kernels/logits_topk.hpp:29-33)."""
    _fields_ = [("v", ctypes.c_float), ("id", ctypes.c_int32)]


class MtpPick(ctypes.Structure):
    """sx_mtp_pick_t: MtpPick (kernels/mtp_pick.hpp:20-28), 64 bytes."""
    _fields_ = [("best", ctypes.c_int32), ("best_v", ctypes.c_float), ("second_v", ctypes.c_float),
                ("nan", ctypes.c_uint32), ("err", ctypes.c_uint32 * 9), ("pad", ctypes.c_uint32),
                ("emb", ctypes.c_ulonglong)]


class StrixwComponentC(ctypes.Structure):
    """sx_strixw_component: StrixwComponent (formats/strixw.hpp:30-33)."""
    _fields_ = [("role", ctypes.c_uint8), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64),
                ("hash", ctypes.c_uint64)]


class StrixwTensorC(ctypes.Structure):
    """sx_strixw_tensor: StrixwTensor (formats/strixw.hpp:35-44)."""
    _fields_ = [("name", ctypes.c_char_p), ("encoding", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 8), ("group_size", ctypes.c_int64), ("experts", ctypes.c_int64),
                ("nparts", ctypes.c_int32), ("ncomp", ctypes.c_int32), ("comp", StrixwComponentC * 4)]


_P, _I64, _INT, _D, _SZP = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.POINTER(ctypes.c_size_t)
_QV = ctypes.POINTER(QView)
_U64, _CP, _PCP = ctypes.c_uint64, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)
_PI64 = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes (restype int unless listed in _RESTYPES). Every symbol include/strixite_amd.h declares.
SIGNATURES = {
    "sx_last_error": [],
    "sx_version": [],
    "sx_linear_q4": [_P, _QV, _P, _I64, _INT, _INT, _P],
    "sx_linear_q8": [_P, _QV, _P, _I64, _INT, _INT, _P],
    "sx_linear_q4_experts_gather": [_P, _QV, _I64, _P, _I64, _I64, _P, _INT, _P, _P],
    "sx_linear_q4_experts_gather_swiglu": [_P, _QV, _I64, _P, _I64, _I64, _P, _INT, _P, _P],
    "sx_linear_q4_experts_combine": [_P, _QV, _I64, _P, _P, _I64, _I64, _P, _INT, _P, _P],
    "sx_report_expert_error": [_P, ctypes.c_char_p],
    "sx_moe_router": [_P, _I64, _I64, _I64, _I64, _P, _I64, ctypes.c_int32, _P, _P, _INT, _P, _P],
    "sx_report_router_error": [_P, ctypes.c_char_p],
    "sx_moe_shared_add": [_P, _P, _P, _I64, _I64, _I64, ctypes.c_uint32, _INT, _P, _P],
    "sx_moe_shared_add_inject": [_P, _P, _P, _I64, _I64, _I64, ctypes.c_uint32, _P, _P, _I64, _INT, _P, _P],
    "sx_moe_route_workspace_bytes": [_I64, _I64, _I64, _SZP],
    "sx_moe_group_routes": [_P, _I64, _I64, _I64, _P, ctypes.c_size_t, _P, _P],
    "sx_linear_q4_experts_gather_grouped": [_P, _QV, _I64, _P, ctypes.c_size_t, _I64, _I64, _P, _INT, _INT, _P],
    "sx_linear_q4_experts_combine_grouped": [_P, _QV, _I64, _P, _P, _P, ctypes.c_size_t, _P, _I64, _I64, _P, _INT,
                                             _INT, _P],
    "sx_linear_q4_experts_gather_swiglu_grouped": [_P, _QV, _I64, _P, ctypes.c_size_t, _I64, _I64, _P, _INT, _P],
    "sx_swiglu": [_P, _P, _I64, _I64, _INT, _P],
    "sx_linear_f32w": [_P, _P, _I64, _I64, _P, _I64, _INT, _P],
    "sx_linear_bf16w": [_P, _P, _P, _I64, _I64, _I64, _INT, _INT, _P],
    "sx_linear_bf16w_wmma": [_P, _P, _P, _I64, _I64, _I64, _INT, _INT, _P],
    "sx_moe_router_group": [_P, _I64, _I64, _I64, _I64, _INT, _P, _P, _P, _P, ctypes.c_size_t, _P, _P],
    "sx_moe_verify_supported": [_I64, _I64, _I64, _I64, _I64, _QV, _QV, _INT],
    "sx_moe_verify_gate_up": [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _INT, _QV, _I64, _P, _P, _P, _P, _INT, _P, _P,
                              _P, _P, _P],
    "sx_moe_verify_down": [_P, _P, _I64, _I64, _P, _P, _QV, _I64, _P, _INT, _P, _P, _P],
    "sx_moe_verify_layer_sync_bytes": [_SZP],
    "sx_moe_verify_layer_trace": [_P],
    "sx_moe_verify_layer": [_P, _I64, _P, _INT, _I64, _I64, _I64, _INT, ctypes.c_int32, _QV, _QV, _I64, _P, _P, _P, _P,
                            _P, _P, _INT, _P, _P, _P, _P],
    "sx_logits_topk_workspace_bytes": [_I64, _I64, _I64, _SZP],
    "sx_logits_topk": [_P, _I64, _I64, _I64, _I64, _P, _P, _P, ctypes.c_size_t, _P, _I64, _P],
    "sx_logits_topk_noalloc": [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P],
    "sx_quantize_q4_from_q8": [_QV, _I64, _P, _P, _P, _P, _P],
    "sx_mtp_pick": [_P, _I64, _P, _P, _P, _P, _P, _P],
    "sx_mtp_pick_ws_bytes": [_I64, _P],
    "sx_mtp_head_pick": [_P, _QV, _INT, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P],
    "sx_mtp_pick_ws": [_P, _I64, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P],
    "sx_mtp_accept": [_P, _P, _I64, _P, _I64, _P, _D, _I64, _D, _I64, _P, _P],
    "sx_strix_hash64": [_P, _U64],
    "sx_strixw_open": [_CP, ctypes.POINTER(_P)],
    "sx_strixw_close": [_P],
    "sx_strixw_summary": [_P, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_U64), ctypes.POINTER(_U64), _PI64,
                          _PI64],
    "sx_strixw_meta_at": [_P, _I64, _PCP, _PCP],
    "sx_strixw_meta": [_P, _CP, _PCP],
    "sx_strixw_find": [_P, _CP, _PI64],
    "sx_strixw_tensor_at": [_P, _I64, ctypes.POINTER(StrixwTensorC)],
    "sx_strixw_part_at": [_P, _I64, _I64, _PCP, _PI64, _PI64],
    "sx_strixw_verify_hashes": [_P, _INT],
    "sx_strixw_load": [_P, _P, _U64, _INT, ctypes.POINTER(_D), _P],
    "sx_strixw_qview": [_P, _P, _CP, _INT, _I64, _I64, _QV],
    "sx_strixw_data": [_P, _P, _CP, _INT, _PI64, _INT, ctypes.POINTER(_P)],
    "sx_verify_tail_workspace_bytes": [_I64, _I64, _I64, _SZP],
    "sx_verify_tail": [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _I64, _P, _D, _I64, _D, _P, _P,
                       ctypes.c_size_t, _P],
    "sx_probe_stream_read": [_P, _U64, _INT, _P, _P],
    "sx_probe_mfma": [_INT, _INT, _P, ctypes.POINTER(_D), _P],
}
_RESTYPES = {"sx_last_error": ctypes.c_char_p, "sx_version": ctypes.c_char_p, "sx_strix_hash64": _U64,
             "sx_strixw_close": None}

_lib = None


def lib():
    """The loaded libstrixite_amd.so (torch is imported first so its HIP runtime is the one the library binds)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m strixite_amd.build` (there is no fallback)")
        try:
            import torch  # noqa: F401  (one HIP runtime in the process: torch's, soname libamdhip64.so.7)
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = L
    return _lib


def check(rc):
    if rc != SX_OK:
        raise SxError(rc, lib().sx_last_error().decode(errors="replace"))
