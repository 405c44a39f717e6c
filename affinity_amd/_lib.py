"""ctypes binding of libaffx.so (include/affx.h). Fails loudly when the library is missing."""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaffx.so")

AFFX_OK = 0
AFFX_DECLINED = 1
AFFX_ROUTE_ENGINE = 0
AFFX_ROUTE_SOFTMAX = 1
AFFX_ERR_ARG = -1
AFFX_ERR_DEVICE = -3

_vp = C.c_void_p
_u32 = C.c_uint32
_u64 = C.c_uint64
_u64p = C.POINTER(C.c_uint64)


class AffxMatrix(C.Structure):
    _fields_ = [("codes", _vp), ("fields", _vp), ("rscales", _vp), ("rows", _u32), ("cols", _u32)]


class AffxExpertTile(C.Structure):
    """affx_expert_tile: one expert matrix's share of a W8A8 GEMM launch (ExpertTile's fields)."""
    _fields_ = [("codes", _vp), ("fields", _vp), ("rscales", _vp), ("tok", _vp), ("y", _vp), ("nt", _u32),
                ("ld", _u32)]


class AffxDeviceExpert(C.Structure):
    _fields_ = [("gate", AffxMatrix), ("up", AffxMatrix), ("down", AffxMatrix)]


class AffxLayer(C.Structure):
    _fields_ = [("base", _vp), ("stride", _u64), ("n_experts", _u32), ("hidden", _u32),
                ("inter", _u32), ("codebook", _vp), ("swiglu_limit", C.c_float)]


class AffxDenseFp8(C.Structure):
    _fields_ = [("data", _vp), ("scales", _vp), ("rows", _u64), ("cols", _u64)]


class AffxSharedExpert(C.Structure):
    _fields_ = [("gate", AffxDenseFp8), ("up", AffxDenseFp8), ("down", AffxDenseFp8), ("hidden", _u32),
                ("inter", _u32), ("swiglu_limit", C.c_float)]


class AffxEngineCtx(C.Structure):
    _fields_ = [("layers", C.POINTER(AffxLayer)), ("n_layers", _u32), ("d_x", _vp),
                ("d_block", _vp), ("nb_stride", _u32), ("workspace", _vp),
                ("workspace_bytes", C.c_size_t), ("stream", _vp)]


class AffxError(RuntimeError):
    pass


class AffxDeclined(AffxError):
    """Preconditions not met, nothing launched (the reference's `false` return)."""


_SIGS = {
    "affx_init": ([], C.c_int),
    "affx_last_error": ([], C.c_char_p),
    "affx_version": ([], C.c_char_p),
    "affx_expert_layout": ([_u64, _u64, _u64p, _u64p], _u64),
    "affx_codebook_valid": ([_vp], C.c_int),
    "affx_expert_to_device_layout": ([_vp, _vp, _u64, _u64], C.c_int),
    "affx_expert_from_device_layout": ([_vp, _vp, _u64, _u64], C.c_int),
    "affx_matrix_to_device_layout": ([_vp, _vp, _vp, _vp, _u32, _u32], C.c_int),
    "affx_expert_ffn": ([C.POINTER(AffxDeviceExpert), _vp, _u32, _vp, _vp, C.c_float, _vp, _vp, _vp], C.c_int),
    "affx_permute_experts": ([_vp, _vp, _u64, _u64, _u64, _vp], C.c_int),
    "affx_container_open": ([C.c_char_p, C.POINTER(_vp)], C.c_int),
    "affx_container_close": ([_vp], None),
    "affx_container_layer_count": ([_vp], _u32),
    "affx_container_layer": ([_vp, _u32, C.POINTER(_u32), _u64p, _u64p, _u64p], C.c_int),
    "affx_container_expert_ptr": ([_vp, _u32, _u32], _vp),
    "affx_container_codebook": ([_vp, _vp], C.c_int),
    "affx_container_upload_layer": ([_vp, _u32, _vp, _vp, _vp], C.c_int),
    "affx_dequant_matrix": ([C.POINTER(AffxMatrix), _vp, _vp, _vp], C.c_int),
    "affx_expert_gemv_batch": ([C.POINTER(AffxMatrix), _vp, _u32, _vp, _vp, _vp, _vp], C.c_int),
    "affx_expert_gemv": ([C.POINTER(AffxMatrix), _vp, _vp, C.c_float, _vp, _vp], C.c_int),
    "affx_decode_workspace_size": ([_u32, _u32, _u32, _u32], C.c_size_t),
    "affx_decode_status": ([_vp, C.c_int, _vp], C.c_int),
    "affx_expert_ffn_decode": ([C.POINTER(AffxLayer), _vp, _u64, _u64, _u32, _vp, _vp, _u32, _vp,
                                _u64, _u64, C.c_int, _vp, C.c_size_t, _vp], C.c_int),
    "affx_expert_ffn_decode_noalloc": ([C.POINTER(AffxLayer), _vp, _u64, _u64, _u32, _vp, _vp, _u32, _vp,
                                        _u64, _u64, C.c_int, _vp], C.c_int),
    "affx_decode_noalloc_status": ([C.c_int, _vp], C.c_int),
    "affx_decode_prepare": ([C.POINTER(AffxLayer), _vp, _u64, _u64, _u32, _vp, _vp, _u32, _vp, C.c_size_t,
                             _vp], C.c_int),
    "affx_decode_gateup": ([C.POINTER(AffxLayer), _u32, _u32, _vp, C.c_size_t, _vp], C.c_int),
    "affx_decode_down": ([C.POINTER(AffxLayer), _u32, _u32, _vp, _u64, _u64, C.c_int, _vp, C.c_size_t, _vp],
                         C.c_int),
    "affx_decode_staged": ([C.POINTER(AffxLayer), _vp, _u64, _u64, _u32, _vp, _vp, _u32, _vp,
                            _u64, _u64, C.c_int, _vp, C.c_size_t, _vp], C.c_int),
    "affx_grouped_workspace_size": ([_u32, _u32, _u32, _u32, _u32], C.c_size_t),
    "affx_expert_ffn_grouped": ([C.POINTER(AffxLayer), _vp, _vp, _u32, _vp, _vp, _u32, _vp, C.c_int,
                                 _vp, C.c_size_t, _vp], C.c_int),
    "affx_expert_ffn_grouped_slots": ([C.POINTER(AffxLayer), _vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _vp,
                                       C.c_int, _vp, C.c_size_t, _vp], C.c_int),
    "affx_expert_swiglu_quant": ([_vp, _vp, _vp, _vp, _vp, _u32, _u32, C.c_float, _vp], C.c_int),
    "affx_expert_scatter_slots": ([_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp], C.c_int),
    "affx_expert_gather_tokens": ([_vp, _vp, _vp, _u32, _u32, _u32, _vp], C.c_int),
    "affx_expert_gemm_w8a8": ([_vp, _u32, _u32, _vp, _vp, _vp, _u32, _u32, C.c_float, C.c_int, _vp], C.c_int),
    "affx_route_topk": ([_vp, _u64, _u64, _vp, _u32, _u32, _u32, C.c_int, C.c_int, C.c_float, _vp, _vp, _vp],
                        C.c_int),
    "affx_dense_fp8_to_device_layout": ([_vp, _vp, _u64, _u64, _vp], C.c_int),
    "affx_shared_decode_workspace_size": ([_u32, _u32, _u32], C.c_size_t),
    "affx_shared_batch_workspace_size": ([_u32, _u32, _u32], C.c_size_t),
    "affx_shared_expert_decode": ([C.POINTER(AffxSharedExpert), _vp, _u64, _u64, _u32, _vp, _u64, _u64, C.c_int,
                                   _vp, C.c_size_t, _vp], C.c_int),
    "affx_shared_expert_batch": ([C.POINTER(AffxSharedExpert), _vp, _vp, _u32, _vp, C.c_int, _vp, C.c_size_t, _vp],
                                 C.c_int),
    "affx_hc_post": ([_vp, _vp, _vp, _vp, _vp, _u32, _u32, C.c_int, _vp], C.c_int),
    "affx_hc_add": ([_vp, _vp, _u32, C.c_int, _vp], C.c_int),
    "affx_hc_post_batch": ([_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, C.c_int, _vp], C.c_int),
    "affx_hc_add_batch": ([_vp, _vp, _u64, C.c_int, _vp], C.c_int),
    "affx_expert_ffn_batch": ([_vp, _u32, _vp, _vp, _u32, _u32, _vp], _u32),
    "affx_batch_workspace_size": ([_u32, _u32, _u32, _u32, _u32], C.c_size_t),
    "affx_selftest_mfma_fp8": ([_vp, _vp, _vp, _vp], C.c_int),
    "affx_gen_normal": ([_u64, _u64, C.c_double, _vp, C.c_int, _vp], C.c_int),
    "affx_quantize_matrix": ([_vp, _u32, _u32, _vp, _vp, _vp, _vp, _vp, _vp], C.c_int),
    "affx_fill_expert": ([_vp, _u64, _u64, _vp, _u32, _vp, _vp], C.c_int),
    "affx_collect_samples_bound": ([_u64, _u64, _u64], _u64),
    "affx_collect_samples_workspace_size": ([_u64, _u64, _u64], C.c_size_t),
    "affx_collect_samples": ([_vp, _u64, _u64, _u64, _vp, _u64, _vp, _vp, C.c_size_t, _vp], C.c_int),
    "affx_fit_codebook_workspace_size": ([_u64], C.c_size_t),
    "affx_fit_codebook": ([_vp, _u64, _vp, _u32, _u64, _u32, _vp, _vp, C.c_size_t, _vp], C.c_int),
    "affx_fit_codebook_stats": ([_vp, _u64p, _u64p, _vp], C.c_int),
    "affx_project_codebook": ([_vp, _u64, _vp], C.c_int),
    "affx_pack_codebook": ([_vp, _vp, _vp], C.c_int),
    "affx_unpack_codebook": ([_vp, _vp, _vp], C.c_int),
}

# every symbol include/affx.h declares (tests check the library exports them all)
HEADER_SYMBOLS = tuple(_SIGS)

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AffxError(f"{LIB_PATH} is missing: build it with `python -m affinity_amd.build` "
                            "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name, None)
            if f is None:
                continue
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def last_error() -> str:
    return lib().affx_last_error().decode(errors="replace")


def check(rc: int, what: str) -> int:
    if rc == AFFX_OK:
        return rc
    if rc == AFFX_DECLINED:
        raise AffxDeclined(f"{what}: {last_error()}")
    raise AffxError(f"{what} failed ({rc}): {last_error()}")
