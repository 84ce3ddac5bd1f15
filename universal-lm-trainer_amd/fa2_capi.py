"""ctypes binding of the C ABI in include/fa2_mi355x.h.

The binding a ctypes-based host writes for this library: struct mirrors of
the parameter blocks and typed entry points.  Used by the tests (direct C-ABI
parity) and by bench.py (per-kernel timing with mode bits 2 and 4)."""
import ctypes
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
HEADER = os.path.join(REPO, "include", "fa2_mi355x.h")
LIB = os.path.join(PKG, "lib", "libfa2_mi355x.so")

I64x3 = ctypes.c_int64 * 3
I64x2 = ctypes.c_int64 * 2


class FwdParams(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("q_stride", I64x3), ("k_stride", I64x3), ("v_stride", I64x3), ("o_stride", I64x3),
        ("lse_stride", I64x2),
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("S", ctypes.c_int32), ("D", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float), ("dropout_p", ctypes.c_float),
        ("seed", ctypes.c_uint32), ("causal", ctypes.c_int32),
        ("dropout_mask", ctypes.c_void_p), ("dropout_mask_bytes", ctypes.c_size_t),
    ]


class BwdParams(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("dout", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("dq", ctypes.c_void_p), ("dk", ctypes.c_void_p), ("dv", ctypes.c_void_p),
        ("q_stride", I64x3), ("k_stride", I64x3), ("v_stride", I64x3), ("o_stride", I64x3),
        ("do_stride", I64x3), ("dq_stride", I64x3), ("dk_stride", I64x3), ("dv_stride", I64x3),
        ("lse_stride", I64x2),
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("S", ctypes.c_int32), ("D", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float), ("dropout_p", ctypes.c_float),
        ("seed", ctypes.c_uint32), ("causal", ctypes.c_int32),
        ("dropout_mask", ctypes.c_void_p), ("dropout_mask_bytes", ctypes.c_size_t),
    ]


class RopeParams(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("qo", ctypes.c_void_p), ("ko", ctypes.c_void_p),
        ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
        ("q_stride", I64x3), ("k_stride", I64x3), ("qo_stride", I64x3), ("ko_stride", I64x3),
        ("cs_stride", ctypes.c_int64), ("sn_stride", ctypes.c_int64),
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("S", ctypes.c_int32), ("D", ctypes.c_int32),
    ]


STRUCTS = {"fa2_fwd_params": FwdParams, "fa2_bwd_params": BwdParams, "fa2_rope_params": RopeParams}


def header_functions():
    """Names of the functions declared in the public header."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(fa2_[a-z0-9_]+)\s*\(", text, re.M)))


_lib = None


def load():
    """Load the C library (torch is imported first so both share one HIP runtime)."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401
        lib = ctypes.CDLL(LIB)
        lib.fa2_fwd_f16.argtypes = [ctypes.POINTER(FwdParams), ctypes.c_void_p]
        lib.fa2_fwd_f16.restype = ctypes.c_int
        lib.fa2_fwd_kv_f16.argtypes = [ctypes.POINTER(FwdParams), ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
        lib.fa2_fwd_kv_f16.restype = ctypes.c_int
        lib.fa2_fwd_kv_split_f16.argtypes = [ctypes.POINTER(FwdParams), ctypes.c_int32, ctypes.c_int32,
                                             ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.fa2_fwd_kv_split_f16.restype = ctypes.c_int
        lib.fa2_fwd_kv_workspace_bytes.argtypes = [ctypes.c_int32] * 4
        lib.fa2_fwd_kv_workspace_bytes.restype = ctypes.c_size_t
        lib.fa2_dropout_mask_bytes.argtypes = [ctypes.c_int32] * 3
        lib.fa2_dropout_mask_bytes.restype = ctypes.c_size_t
        lib.fa2_dropout_mask_bytes_causal.argtypes = [ctypes.c_int32] * 3
        lib.fa2_dropout_mask_bytes_causal.restype = ctypes.c_size_t
        lib.fa2_dropout_threshold.argtypes = [ctypes.c_float]
        lib.fa2_dropout_threshold.restype = ctypes.c_uint32
        lib.fa2_bwd_f16.argtypes = [ctypes.POINTER(BwdParams), ctypes.c_int32, ctypes.c_void_p,
                                    ctypes.c_size_t, ctypes.c_void_p]
        lib.fa2_bwd_f16.restype = ctypes.c_int
        lib.fa2_bwd_workspace_bytes.argtypes = [ctypes.c_int32] * 3
        lib.fa2_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.fa2_bwd_f16_noalloc.argtypes = [ctypes.POINTER(BwdParams), ctypes.c_int32, ctypes.c_void_p]
        lib.fa2_bwd_f16_noalloc.restype = ctypes.c_int
        lib.fa2_bwd_noalloc_scratch_bytes.argtypes = [ctypes.c_int32] * 3
        lib.fa2_bwd_noalloc_scratch_bytes.restype = ctypes.c_size_t
        lib.fa2_rope_f16.argtypes = [ctypes.POINTER(RopeParams), ctypes.c_int32, ctypes.c_void_p]
        lib.fa2_rope_f16.restype = ctypes.c_int
        lib.fa2_status_string.argtypes = [ctypes.c_int]
        lib.fa2_status_string.restype = ctypes.c_char_p
        lib.fa2_last_error.argtypes = []
        lib.fa2_last_error.restype = ctypes.c_char_p
        lib.fa2_version.argtypes = []
        lib.fa2_version.restype = ctypes.c_char_p
        _lib = lib
    return _lib


def strides3(t):
    return I64x3(t.stride(0), t.stride(1), t.stride(2))


def fwd_params(q, k, v, o, lse, scale, causal=True, dropout_p=0.0, seed=0, mask=None):
    p = FwdParams()
    p.dropout_mask = mask.data_ptr() if mask is not None else None
    p.dropout_mask_bytes = mask.numel() * mask.element_size() if mask is not None else 0
    p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    p.q_stride, p.k_stride, p.v_stride, p.o_stride = strides3(q), strides3(k), strides3(v), strides3(o)
    p.lse_stride = I64x2(lse.stride(0), lse.stride(1))
    p.B, p.H, p.S, p.D = q.size(0), q.size(1), q.size(2), q.size(3)
    p.softmax_scale, p.dropout_p, p.seed, p.causal = scale, dropout_p, seed, int(causal)
    return p


def bwd_params(q, k, v, o, lse, do, dq, dk, dv, scale, causal=True, dropout_p=0.0, seed=0, mask=None):
    p = BwdParams()
    p.dropout_mask = mask.data_ptr() if mask is not None else None
    p.dropout_mask_bytes = mask.numel() * mask.element_size() if mask is not None else 0
    p.q, p.k, p.v, p.o, p.dout = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr()
    p.lse, p.dq, p.dk, p.dv = lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    p.q_stride, p.k_stride, p.v_stride = strides3(q), strides3(k), strides3(v)
    p.o_stride, p.do_stride = strides3(o), strides3(do)
    p.dq_stride, p.dk_stride, p.dv_stride = strides3(dq), strides3(dk), strides3(dv)
    p.lse_stride = I64x2(lse.stride(0), lse.stride(1))
    p.B, p.H, p.S, p.D = q.size(0), q.size(1), q.size(2), q.size(3)
    p.softmax_scale, p.dropout_p, p.seed, p.causal = scale, dropout_p, seed, int(causal)
    return p


def rope_params(q, k, qo, ko, cos, sin):
    p = RopeParams()
    p.q, p.k, p.qo, p.ko = q.data_ptr(), k.data_ptr(), qo.data_ptr(), ko.data_ptr()
    p.cos, p.sin = cos.data_ptr(), sin.data_ptr()
    p.q_stride, p.k_stride, p.qo_stride, p.ko_stride = strides3(q), strides3(k), strides3(qo), strides3(ko)
    p.cs_stride, p.sn_stride = cos.stride(0), sin.stride(0)
    p.B, p.H, p.S, p.D = q.size(0), q.size(1), q.size(2), q.size(3)
    return p
