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
            "ssdo_rope_multi_head": (None, [_vp, _sz, _sz, _sz, _sz, ctypes.c_float]),
            "ssdo_kv_slot_bytes": (_sz, [_sz, _sz]),
            "ssdo_kv_swap_write": (None, [_vp, _vp, _sz, _sz, ctypes.c_uint32, _vp]),
            "ssdo_kv_swap_read": (None, [_vp, _sz, _sz, _vp, _vp, _vp]),
            "ssdo_silu": (None, [_vp, _sz]),
            "ssdo_rmsnorm": (None, [_vp, _vp, _sz, ctypes.c_float]),
            "ssdo_fused_post_attn_norm": (None, [_vp, _vp, _vp, _sz, ctypes.c_float, _vp]),
            "ssdo_fused_rmsnorm_linear": (_i, [_i, _vp, _vp, _vp, _sz, _sz, _vp]),
            "ssdo_quantize_rows_int8": (None, [_vp, _sz, _sz, _vp, _vp]),
            "ssdo_dequantize_rows_int8": (None, [_vp, _vp, _sz, _sz, _vp]),
            "ssdo_flash_attention_f32": (None, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
            "ssdo_paged_attention_int8_mt": (
                None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _i]),
            "ssdo_paged_attention_int8_window_mt": (
                None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _i]),
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


def paged_attention_int8_window(q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, window_starts,
                                window_ends, n_seq, n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq,
                                threads=1):
    """paged_attention_int8 over [window_starts[s], min(window_ends[s], ctx_lens[s])) per sequence
    (flash_attention_windowed, src/inference/flash_attention.rs:146-227); either may be None."""
    q = _c(q, np.float32)
    kc, vc = _c(k_codes, np.int8), _c(v_codes, np.int8)
    ks, vs = _c(k_scales, np.float32), _c(v_scales, np.float32)
    bt, cl = _c(block_tables, np.int32), _c(ctx_lens, np.int32)
    lo = None if window_starts is None else _c(window_starts, np.int32)
    hi = None if window_ends is None else _c(window_ends, np.int32)
    out = np.empty(n_seq * n_head * head_dim, np.float32)
    lib().ssdo_paged_attention_int8_window_mt(q.ctypes.data, kc.ctypes.data, ks.ctypes.data, vc.ctypes.data,
                                              vs.ctypes.data, bt.ctypes.data, cl.ctypes.data,
                                              None if lo is None else lo.ctypes.data,
                                              None if hi is None else hi.ctypes.data, n_seq, n_head, n_head_kv,
                                              head_dim, block_size, max_blocks_per_seq, out.ctypes.data, threads)
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


def rope_multi_head(x, head_dim, n_heads, position, theta_base):
    x = np.array(x, np.float32)
    lib().ssdo_rope_multi_head(x.ctypes.data, x.size, head_dim, n_heads, position, theta_base)
    return x


def silu(x):
    x = np.array(x, np.float32)
    lib().ssdo_silu(x.ctypes.data, x.size)
    return x


def rmsnorm(x, w, eps):
    x = np.array(x, np.float32)
    w = _c(w, np.float32)
    lib().ssdo_rmsnorm(x.ctypes.data, w.ctypes.data, x.size, eps)
    return x


def fused_post_attn_norm(hidden, attn, w, eps):
    """(hidden after the residual add, normalized output)"""
    hidden = np.array(hidden, np.float32)
    attn = _c(attn, np.float32)
    w = _c(w, np.float32)
    out = np.empty_like(hidden)
    lib().ssdo_fused_post_attn_norm(hidden.ctypes.data, attn.ctypes.data, w.ctypes.data, hidden.size,
                                    eps, out.ctypes.data)
    return hidden, out


def fused_rmsnorm_linear(dtype, w, x, norm_w, vocab, n_embd):
    w = _c(w, np.uint8)
    x = _c(x, np.float32)
    norm_w = _c(norm_w, np.float32)
    y = np.empty(vocab, np.float32)
    rc = lib().ssdo_fused_rmsnorm_linear(dtype, w.ctypes.data, x.ctypes.data, norm_w.ctypes.data,
                                         vocab, n_embd, y.ctypes.data)
    return y, rc


def qkv_rope(dq, wq, dk, wk, dv, wv, x, q_dim, kv_dim, n_embd, head_dim, position, theta):
    """fused_qkv_rope_f32_cpu (compute.rs:509-534) with the projections through
    matvec_quantized_cpu; head_dim 0 leaves out the rotation (fused_qkv_f32_cpu)."""
    q, _ = matvec(dq, wq, x, q_dim, n_embd)
    k, _ = matvec(dk, wk, x, kv_dim, n_embd)
    v, _ = matvec(dv, wv, x, kv_dim, n_embd)
    if head_dim:
        q = rope_multi_head(q, head_dim, q_dim // head_dim, position, theta)
        k = rope_multi_head(k, head_dim, kv_dim // head_dim, position, theta)
    return q, k, v


def swiglu(dtype, w_gate, w_up, x, n_ff, n_embd):
    """silu(W_gate x) * (W_up x), feed_forward.rs:28-40 with matvec_quantized_cpu."""
    g, _ = matvec(dtype, w_gate, x, n_ff, n_embd)
    g = silu(g)
    u, _ = matvec(dtype, w_up, x, n_ff, n_embd)
    return (g * u).astype(np.float32)


def kv_slot_bytes(block_size, kv_dim):
    return lib().ssdo_kv_slot_bytes(block_size, kv_dim)


def kv_swap_write(keys, values, block_size, kv_dim, num_filled):
    keys = _c(keys, np.float32)
    values = _c(values, np.float32)
    slot = np.zeros(kv_slot_bytes(block_size, kv_dim), np.uint8)
    lib().ssdo_kv_swap_write(keys.ctypes.data, values.ctypes.data, block_size, kv_dim, num_filled,
                             slot.ctypes.data)
    return slot


def kv_swap_read(slot, block_size, kv_dim):
    slot = _c(slot, np.uint8)
    k = np.empty(block_size * kv_dim, np.float32)
    v = np.empty(block_size * kv_dim, np.float32)
    nf = np.zeros(1, np.uint32)
    lib().ssdo_kv_swap_read(slot.ctypes.data, block_size, kv_dim, k.ctypes.data, v.ctypes.data, nf.ctypes.data)
    return k, v, int(nf[0])
