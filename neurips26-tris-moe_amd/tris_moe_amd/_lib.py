"""ctypes binding of libtris_moe_hip.so (the C ABI declared in include/tris_moe_hip.h).

The library is built in place by ``make -C neurips26-tris-moe_amd`` (or
``__graft_entry__.build()``).  Loading fails loudly: there is no CPU or torch
fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("TRIS_MOE_HIP_LIB", PKG_ROOT / "libtris_moe_hip.so"))

TRIS_COMPACT3_KERNEL_ABI_VERSION = 2


class TrisExtensionUnavailable(ImportError):
    """The HIP library is missing or incompatible."""


class TrisPayload(ctypes.Structure):
    """Mirror of struct tris_compact3_payload."""

    _fields_ = [
        ("num_experts", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("outfeatures", ctypes.c_int32),
        ("num_groups", ctypes.c_int32),
        ("qweight2_sparse_rows", ctypes.c_int32),
        ("gr_words_stride", ctypes.c_int32),
        ("qweight1", ctypes.c_void_p),
        ("qweight2_sparse", ctypes.c_void_p),
        ("qweight2_sparse_prefix", ctypes.c_void_p),
        ("q_gmap_gr_words", ctypes.c_void_p),
        ("q_gmap_gr_offsets", ctypes.c_void_p),
        ("q_gmap_gr_meta", ctypes.c_void_p),
        ("c_map", ctypes.c_void_p),
        ("g_idx", ctypes.c_void_p),
        ("col_pack3", ctypes.c_void_p),
        ("row_pack3", ctypes.c_void_p),
        ("output_scale", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("has_output_scale", ctypes.c_int32),
        ("has_bias", ctypes.c_int32),
        ("use_uniform_k64_groups", ctypes.c_int32),
    ]


# name -> (restype, argtypes)
class TrisPredecodeJob(ctypes.Structure):
    """Mirror of struct tris_gr_predecode_job."""

    _fields_ = [
        ("decoded", ctypes.c_void_p),
        ("q_gmap_gr_words", ctypes.c_void_p),
        ("q_gmap_gr_offsets", ctypes.c_void_p),
        ("q_gmap_gr_meta", ctypes.c_void_p),
        ("num_experts", ctypes.c_int32),
        ("words_stride", ctypes.c_int32),
        ("packed_rows", ctypes.c_int32),
        ("outfeatures", ctypes.c_int32),
    ]


class TrisBackbonePairJob(ctypes.Structure):
    """Mirror of struct tris_backbone_pair_job."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("tokens", ctypes.c_int32),
        ("in_features", ctypes.c_int32),
        ("sv_a", ctypes.c_void_p),
        ("sv_b", ctypes.c_void_p),
        ("rank", ctypes.c_int32),
        ("in_scale_a", ctypes.c_void_p),
        ("in_scale_b", ctypes.c_void_p),
        ("out_a", ctypes.c_void_p),
        ("out_b", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("out_a_hi", ctypes.c_void_p),
        ("out_b_hi", ctypes.c_void_p),
        ("split", ctypes.c_int32),
    ]


class TrisPacked4(ctypes.Structure):
    """Mirror of struct tris_packed4_matrix."""

    _fields_ = [
        ("qweight", ctypes.c_void_p),
        ("qzeros", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("g_idx", ctypes.c_void_p),
        ("rows", ctypes.c_int32),
        ("cols", ctypes.c_int32),
        ("num_groups", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
    ]


class TrisNsPayload(ctypes.Structure):
    """Mirror of struct tris_ns_payload."""

    _fields_ = [
        ("ns_rank_per_expert", ctypes.c_void_p),
        ("ns_c2_rank_offsets", ctypes.c_void_p),
        ("ns_c2_rank_word_offsets", ctypes.c_void_p),
        ("ns_c1_rank_word_offsets", ctypes.c_void_p),
        ("ns_c1_group_offsets", ctypes.c_void_p),
        ("ns_c2_qweight", ctypes.c_void_p),
        ("ns_c2_qzeros", ctypes.c_void_p),
        ("ns_c2_scales", ctypes.c_void_p),
        ("ns_c1_qweight", ctypes.c_void_p),
        ("ns_c1_qzeros", ctypes.c_void_p),
        ("ns_c1_scales", ctypes.c_void_p),
        ("num_experts", ctypes.c_int32),
        ("infeatures", ctypes.c_int32),
        ("outfeatures", ctypes.c_int32),
        ("max_ns_rank", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("total_rank", ctypes.c_int32),
        ("total_rank_words", ctypes.c_int32),
    ]


MAX_PREDECODE_JOBS = 4

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_PAY = ctypes.POINTER(TrisPayload)
_P4 = ctypes.POINTER(TrisPacked4)
_PNS = ctypes.POINTER(TrisNsPayload)
SIGNATURES = {
    "tris_abi_version": (ctypes.c_int, []),
    "tris_last_error": (ctypes.c_char_p, []),
    "tris_gr_encode": (_I64, [_P, _I32, _I32, _I32, _I32, _I32, _P, _I64, _P, _P]),
    "tris_build_grouped_route": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "tris_route_topk_grouped": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                _P, _P, _P, _P]),
    "tris_grouped_forward_block_gr": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I32, _I64, _PAY, _P, _P]),
    "tris_route_topk": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _P, _P, _P, _P]),
    "tris_grouped_forward_sparse": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I32, _I64, _PAY, _P, _P, _I32, _P, _P]),
    "tris_grouped_decode_forward_block_gr": (ctypes.c_int, [_P, _P, _I32, _I32, _P, _P, _I32, _PAY, _P, _P]),
    "tris_grouped_decode_pair_forward_block_gr": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _P, _P, _I32, _PAY, _PAY,
                                                                 _P, _P, _I32, _P]),
    "tris_grouped_dual_forward_block_gr": (ctypes.c_int, [_P, _P, _I32, _P, _P, _P, _I32, _I64, _PAY, _PAY, _P, _P, _P]),
    "tris_grouped_block_gr_predecode": (ctypes.c_int, [_P, _P, _I32, _P, _P, _P, _I32, _I32, _I32, _I32, _P]),
    "tris_grouped_block_gr_predecode_multi": (ctypes.c_int, [ctypes.POINTER(TrisPredecodeJob), _I32, _P, _I32, _P]),
    "tris_grouped_block_gr_predecode_multi_reduce": (
        ctypes.c_int, [ctypes.POINTER(TrisPredecodeJob), _I32, _P, _I32, ctypes.POINTER(TrisBackbonePairJob), _P]),
    "tris_route_topk_backbone": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                 _P, _P, _P, ctypes.POINTER(TrisBackbonePairJob), _I32, _P]),
    "tris_grouped_forward_block_gr_predecoded": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I32, _I64, _P, _PAY, _P, _P]),
    "tris_grouped_dual_forward_block_gr_predecoded": (
        ctypes.c_int, [_P, _P, _I32, _P, _P, _P, _I32, _I64, _P, _P, _PAY, _PAY, _P, _P, _P]),
    "tris_grouped_swiglu_forward_block_gr_predecoded": (
        ctypes.c_int, [_P, _P, _I32, _P, _P, _P, _I32, _I64, _P, _P, _PAY, _PAY, _P, _P]),
    "tris_grouped_dual_forward_block_gr_predecoded_rows": (
        ctypes.c_int, [_P, _P, _P, _I32, _I32, _P, _P, _I32, _I64, _P, _P, _PAY, _PAY, _P, _P, _P]),
    "tris_grouped_swiglu_forward_block_gr_predecoded_rows": (
        ctypes.c_int, [_P, _P, _P, _I32, _I32, _P, _P, _I32, _I64, _P, _P, _PAY, _PAY, _P, _P]),
    "tris_compact3_dequant": (ctypes.c_int, [_PAY, _P, _I32, _P, _P]),
    "tris_gr_decode_dense": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _P, _I32, _I32, _I32, _P, _P]),
    "tris_backbone_linear": (ctypes.c_int, [_P, _I32, _I32, _P, _P, _I32, _P, _P, _P, _I64, _P]),
    "tris_backbone_linear_deferred": (ctypes.c_int, [_P, _I32, _I32, _P, _P, _I32, _P, _P, _P, _I64, _P, _P]),
    "tris_backbone_linear_pair": (ctypes.c_int, [_P, _I32, _I32, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _I64, _P]),
    "tris_backbone_pair_workspace_bytes": (_I64, [_I32, _I32, _I32]),
    "tris_backbone_swiglu_linear": (ctypes.c_int, [_P, _P, _I32, _I32, _P, _I32, _P, _P, _P, _I64, _P]),
    "tris_backbone_swiglu_linear_split": (ctypes.c_int, [_P, _P, _I32, _I32, _P, _I32, _P, _P, _P, _I32, _P, _I64,
                                                         _P]),
    "tris_backbone_swiglu_workspace_bytes": (_I64, [_I32, _I32, _I32]),
    "tris_backbone_linear_pair_scatter": (ctypes.c_int, [_P, _I32, _I32, _P, _P, _I32, _P, _P, _P, _I32, _I32, _P, _P,
                                                          _P, _I64, _P]),
    "tris_backbone_scatter_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32]),
    "tris_backbone_linear_noalloc": (ctypes.c_int, [_P, _I32, _I32, _P, _P, _I32, _P, _P, _P]),
    "tris_backbone_noalloc_scratch_bytes": (_I64, []),
    "tris_backbone_workspace_bytes": (_I64, [_I32, _I32, _I32]),
    "tris_moe_combine": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I32, _I32, _P, _P]),
    "tris_moe_combine_compensated": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _P, _P]),
    "tris_router_linear": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _I32, _P, _P, _P, _P]),
    "tris_router_backbone": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _P, _P, _P,
                                            ctypes.POINTER(TrisBackbonePairJob), _P]),
    "tris_route_predecode_multi_reduce": (
        ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                       ctypes.POINTER(TrisPredecodeJob), _I32, _I32, ctypes.POINTER(TrisBackbonePairJob), _P]),
    "tris_route_predecode_all_reduce": (
        ctypes.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                       ctypes.POINTER(TrisPredecodeJob), _I32, ctypes.POINTER(TrisBackbonePairJob), _P]),
    "tris_grouped_forward_block_gr_predecoded_experts": (
        ctypes.c_int, [_P, _P, _P, _I32, _I32, _P, _P, _I32, _I64, _P, _P, _PAY, _PAY, _P, _P, _P]),
    "tris_grouped_forward_block_gr_predecoded_partials": (
        ctypes.c_int, [_P, _I32, _I32, _P, _P, _I32, _I64, _P, _PAY, _P, _I32, _P]),
    "tris_grouped_forward_block_gr_predecoded_partials_combine": (
        ctypes.c_int, [_P, _I32, _P, _P, _I64, _P, _PAY, _P, _P, _I32, _P, _I32, _P]),
    "tris_moe_combine_gated": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _P, _P]),
    "tris_swiglu_mul": (ctypes.c_int, [_P, _P, _I64, _P, _P]),
    "tris_swiglu_mul_compensated": (ctypes.c_int, [_P, _P, _P, _P, _I64, _P, _P]),
    "tris_packed4_dequant": (ctypes.c_int, [_P4, _P, _P]),
    "tris_packed4_backbone_linear": (ctypes.c_int, [_P, _I32, _P, _P4, _P, _P, _P, _I64, _P]),
    "tris_packed4_backbone_linear_pair": (ctypes.c_int, [_P, _I32, _P, _P4, _P4, _P, _P, _P, _P, _P, _I64, _P]),
    "tris_grouped_ns_compensation_forward": (ctypes.c_int, [_P, _I32, _P, _P, _I32, _PNS, _P, _I64, _P, _I32, _P]),
    "tris_grouped_ns_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32]),
    "tris_grouped_ns_compensation_pair_forward": (ctypes.c_int, [_P, _I32, _P, _I32, _P, _P, _I32, _PNS, _PNS, _P, _I64,
                                                                 _P, _P, _I32, _P]),
    "tris_grouped_ns_pair_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I32]),
    "tris_grouped_ns_c1_forward": (ctypes.c_int, [_P, _I32, _P, _P, _I32, _PNS, _P, _I32, _P]),
    "tris_compact3_linear_forward": (ctypes.c_int, [_P, _I32, _PAY, _P, _P, _P, _P]),
    "tris_compact3_dual_linear_forward": (ctypes.c_int, [_P, _I32, _PAY, _PAY, _P, _P, _P]),
    "tris_dense_linear_f32": (ctypes.c_int, [_P, _P, _I32, _I32, _P, _I32, _P, _P]),
}

_lib = None


def load():
    """Load and type the HIP library (cached).  Raises TrisExtensionUnavailable."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise TrisExtensionUnavailable(
            f"TriS HIP library not found at {LIB_PATH}; build it with `make -C {PKG_ROOT}` "
            "(there is no CPU fallback)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    missing = [name for name in SIGNATURES if not hasattr(lib, name)]
    if missing:
        raise TrisExtensionUnavailable(f"{LIB_PATH} lacks entry points {missing}; rebuild it")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    version = lib.tris_abi_version()
    if version != TRIS_COMPACT3_KERNEL_ABI_VERSION:
        raise TrisExtensionUnavailable(
            f"{LIB_PATH}: compact3 ABI {version}, expected {TRIS_COMPACT3_KERNEL_ABI_VERSION}")
    _lib = lib
    return lib


def check(rc: int, what: str):
    """Turn a negative C-ABI return code into RuntimeError (the reference's TORCH_CHECK)."""
    if rc < 0:
        msg = load().tris_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{what}: {msg}")
    return rc
