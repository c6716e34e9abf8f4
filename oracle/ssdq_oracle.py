"""ctypes wrapper of the CPU oracle (libssdq_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product library never loads it.  numpy arrays in, numpy arrays out.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libssdq_oracle.so")

_lib = None
_vp, _sz, _i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        l = ctypes.CDLL(LIB_PATH)
        sig = {
            "ssdo_block_size": (_sz, [_i]),
            "ssdo_type_size": (_sz, [_i]),
            "ssdo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "ssdo_f16_to_f32_array": (None, [_vp, _sz, _vp]),
            "ssdo_dequantize_to_f32": (_i, [_i, _vp, _sz, _sz, _vp]),
            "ssdo_matvec_quantized": (_i, [_vp, _vp, _sz, _sz, _i, _vp]),
            "ssdo_matvec_quantized_mt": (_i, [_vp, _vp, _sz, _sz, _i, _vp, _i]),
            "ssdo_matvec_exact": (_i, [_vp, _vp, _sz, _sz, _i, _vp]),
            "ssdo_matvec_elements": (_i, [_vp, _sz, _sz, _i, _vp]),
            "ssdo_quantize_rows_int8": (None, [_vp, _sz, _sz, _vp, _vp]),
            "ssdo_dequantize_rows_int8": (None, [_vp, _vp, _sz, _sz, _vp]),
            "ssdo_flash_attention_f32": (None, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
            "ssdo_paged_attention_int8_mt": (
                None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _i]),
            "ssdo_gemm_q4k_bf16": (None, [_vp, _vp, _sz, _sz, _sz, _vp, _i]),
            "ssdo_gemm_q4k_bf16_exact": (None, [_vp, _vp, _sz, _sz, _sz, _vp, _i]),
        }
        for name, (res, args) in sig.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def block_size(dtype):
    return lib().ssdo_block_size(dtype)


def type_size(dtype):
    return lib().ssdo_type_size(dtype)


def f16_to_f32(bits):
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().ssdo_f16_to_f32_array(bits.ctypes.data, bits.size, out.ctypes.data)
    return out


def dequantize(dtype, data, n_elements):
    data = _c(data, np.uint8)
    out = np.empty(n_elements, np.float32)
    rc = lib().ssdo_dequantize_to_f32(dtype, data.ctypes.data, data.size, n_elements, out.ctypes.data)
    return out, rc


def matvec(dtype, w, x, out_dim, in_dim, threads=1):
    w = _c(w, np.uint8)
    x = _c(x, np.float32)
    y = np.empty(out_dim, np.float32)
    if threads > 1:
        rc = lib().ssdo_matvec_quantized_mt(w.ctypes.data, x.ctypes.data, out_dim, in_dim, dtype,
                                            y.ctypes.data, threads)
    else:
        rc = lib().ssdo_matvec_quantized(w.ctypes.data, x.ctypes.data, out_dim, in_dim, dtype,
                                         y.ctypes.data)
    return y, rc


def matvec_exact(dtype, w, x, out_dim, in_dim):
    w = _c(w, np.uint8)
    x = _c(x, np.float32)
    y = np.empty(out_dim, np.float64)
    lib().ssdo_matvec_exact(w.ctypes.data, x.ctypes.data, out_dim, in_dim, dtype, y.ctypes.data)
    return y


def matvec_elements(dtype, w, out_dim, in_dim):
    """The element values each matvec multiplies by x, [out_dim, whole blocks of in_dim]."""
    w = _c(w, np.uint8)
    k = (in_dim // block_size(dtype)) * block_size(dtype)
    e = np.zeros((out_dim, k), np.float32)
    rc = lib().ssdo_matvec_elements(w.ctypes.data, out_dim, in_dim, dtype, e.ctypes.data)
    return e, rc


def quantize_rows(data, n_rows, dim):
    data = _c(data, np.float32)
    codes = np.empty(n_rows * dim, np.int8)
    scales = np.empty(n_rows, np.float32)
    lib().ssdo_quantize_rows_int8(data.ctypes.data, n_rows, dim, codes.ctypes.data, scales.ctypes.data)
    return codes, scales


def dequantize_rows(codes, scales, n_rows, dim):
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    out = np.empty(n_rows * dim, np.float32)
    lib().ssdo_dequantize_rows_int8(codes.ctypes.data, scales.ctypes.data, n_rows, dim, out.ctypes.data)
    return out


def flash_attention_f32(q, k, v, n_head, n_head_kv, head_dim, seq_len, window_start, window_end):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    out = np.empty(n_head * head_dim, np.float32)
    lib().ssdo_flash_attention_f32(q.ctypes.data, k.ctypes.data, v.ctypes.data, n_head, n_head_kv,
                                   head_dim, seq_len, window_start, window_end, out.ctypes.data)
    return out


def paged_attention_int8(q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, n_seq,
                         n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq, threads=1):
    q = _c(q, np.float32)
    kc, vc = _c(k_codes, np.int8), _c(v_codes, np.int8)
    ks, vs = _c(k_scales, np.float32), _c(v_scales, np.float32)
    bt, cl = _c(block_tables, np.int32), _c(ctx_lens, np.int32)
    out = np.empty(n_seq * n_head * head_dim, np.float32)
    lib().ssdo_paged_attention_int8_mt(q.ctypes.data, kc.ctypes.data, ks.ctypes.data, vc.ctypes.data,
                                       vs.ctypes.data, bt.ctypes.data, cl.ctypes.data, n_seq, n_head,
                                       n_head_kv, head_dim, block_size, max_blocks_per_seq,
                                       out.ctypes.data, threads)
    return out


def gemm_q4k_bf16(w, x_bf16, M, N, K, threads=1, exact=False):
    w = _c(w, np.uint8)
    x = _c(x_bf16, np.uint16)
    if exact:
        y = np.empty(M * N, np.float64)
        lib().ssdo_gemm_q4k_bf16_exact(w.ctypes.data, x.ctypes.data, M, N, K, y.ctypes.data, threads)
    else:
        y = np.empty(M * N, np.float32)
        lib().ssdo_gemm_q4k_bf16(w.ctypes.data, x.ctypes.data, M, N, K, y.ctypes.data, threads)
    return y
