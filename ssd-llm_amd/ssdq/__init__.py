"""ctypes binding of libssdq.so (the C ABI declared in include/ssdq.h).

This is plumbing for tests and benchmarks: device buffers and streams come
from PyTorch, the compute is the HIP library.  Every call goes through the
C ABI and raises SsdqError on a negative status; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_ROOT, "libssdq.so")

# GgmlType ids, src/model/gguf.rs:17-48
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 14, 30
Q2_K, Q3_K, Q5_K, Q8_K, IQ4_NL, IQ4_XS = 10, 11, 13, 15, 20, 23
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S = 16, 17, 18, 21
# dequant (streamer.rs:93-125) and the prefill path cover these four
QUANT_TYPES = (Q4_0, Q8_0, Q4_K, Q6_K)
# the other matvec_quantized types (compute.rs:655-671)
MATVEC_EXTRA_TYPES = (Q2_K, Q3_K, Q5_K, Q8_K, IQ4_NL, IQ4_XS, F16, BF16, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S)
TYPE_NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", Q2_K: "Q2_K", Q3_K: "Q3_K",
              Q5_K: "Q5_K", Q8_K: "Q8_K", IQ4_NL: "IQ4_NL", IQ4_XS: "IQ4_XS", F16: "F16",
              BF16: "BF16", IQ2_XXS: "IQ2_XXS", IQ2_XS: "IQ2_XS", IQ3_XXS: "IQ3_XXS", IQ3_S: "IQ3_S"}

OK = 0
WARN_UNSUPPORTED_ZEROED = 1


class SsdqError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


_c = ctypes
_vp, _sz, _i = _c.c_void_p, _c.c_size_t, _c.c_int



class LayerConfig(ctypes.Structure):
    """ssdq_layer_config: one decoder layer's shape."""
    _fields_ = [("n_embd", _sz), ("n_head", _sz), ("n_head_kv", _sz), ("head_dim", _sz), ("n_ff", _sz),
                ("rope_theta", _c.c_float), ("norm_eps", _c.c_float)]


# scratch regions of ssdq_decode_layer_dev (SSDQ_LAYER_*)
LAYER_STAGES = ("attn_in", "q", "k", "v", "attn", "attn_out", "ffn_in", "ffn_h", "ffn_gate", "ffn_up",
                "ffn_out", "norm_w", "hidden_mid")

_u64p = _c.POINTER(_c.c_uint64)

# name -> (restype, argtypes); mirrors include/ssdq.h
SIGNATURES = {
    "ssdq_abi_version": (_i, []),
    "ssdq_last_error": (_c.c_char_p, []),
    "ssdq_block_size": (_sz, [_i]),
    "ssdq_type_size": (_sz, [_i]),
    "ssdq_row_bytes": (_sz, [_i, _sz]),
    "ssdq_ctx_create": (_i, [_i, _c.POINTER(_vp)]),
    "ssdq_ctx_destroy": (None, [_vp]),
    "ssdq_ctx_device": (_i, [_vp]),
    "ssdq_reserve_workspace": (_i, [_sz, _vp]),
    "ssdq_release_workspaces": (_i, []),
    "ssdq_dequant_dev": (_i, [_i, _vp, _sz, _vp, _vp]),
    "ssdq_matvec_dev": (_i, [_i, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "ssdq_matvec_generic_dev": (_i, [_i, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "ssdq_matvec_quantized": (_i, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _i, _vp]),
    "ssdq_gemm_q4k_bf16_dev": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "ssdq_gemm_q4k_bf16_multi_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _vp]),
    "ssdq_kv_slot_bytes": (_sz, [_sz, _sz]),
    "ssdq_kv_swap_out_dev": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _vp]),
    "ssdq_kv_swap_in_dev": (_i, [_vp, _vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ssdq_qkv_rope_dev": (_i, [_i, _vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz,
                               _c.c_float, _vp]),
    "ssdq_swiglu_dev": (_i, [_i, _vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "ssdq_rmsnorm_matvec_dev": (_i, [_i, _vp, _vp, _vp, _c.c_float, _vp, _sz, _sz, _vp]),
    "ssdq_rmsnorm_dev": (_i, [_vp, _vp, _vp, _c.c_float, _vp, _vp, _sz, _vp]),
    "ssdq_kv_quantize_rows_dev": (_i, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "ssdq_kv_dequantize_rows_dev": (_i, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "ssdq_paged_kv_append_dev": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "ssdq_paged_attention_int8_dev": (
        _i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
    "ssdq_paged_attention_int8_window_dev": (
        _i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
    "ssdq_paged_attention_int8_noalloc_dev": (
        _i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
    "ssdq_flash_attention_f32_dev": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
    "ssdq_flash_attention_f32": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
    "ssdq_dequantize_to_f32": (_i, [_vp, _i, _vp, _sz, _sz, _vp]),
    "ssdq_quantize_vectors_int8": (_i, [_vp, _vp, _sz, _sz, _vp, _vp]),
    "ssdq_dequantize_vectors_int8": (_i, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "ssdq_weights_create": (_i, [_i, _c.POINTER(_vp)]),
    "ssdq_weights_destroy": (None, [_vp]),
    "ssdq_weights_put": (_i, [_vp, _c.c_char_p, _i, _u64p, _sz, _vp, _sz]),
    "ssdq_weights_find": (_vp, [_vp, _c.c_char_p, _c.POINTER(_i), _u64p, _c.POINTER(_sz), _c.POINTER(_sz)]),
    "ssdq_weights_count": (_sz, [_vp]),
    "ssdq_weights_bytes": (_sz, [_vp]),
    "ssdq_weights_device": (_i, [_vp]),
    "ssdq_decode_layer_scratch_bytes": (_sz, [_c.POINTER(LayerConfig), _c.POINTER(_sz)]),
    "ssdq_decode_layer_dev": (_i, [_vp, _c.c_uint32, _c.POINTER(LayerConfig), _vp, _sz, _vp, _vp, _vp, _vp, _sz,
                                   _vp, _sz, _vp, _vp, _sz, _vp, _sz, _vp]),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libssdq.so (built in-tree by __graft_entry__.build()); raises if absent."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise FileNotFoundError(
                    f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
            l = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                f = getattr(l, name)
                f.restype = res
                f.argtypes = args
            _lib = l
    return _lib


def last_error() -> str:
    return (lib().ssdq_last_error() or b"").decode()


def check(fn: str, rc: int) -> int:
    if rc < 0:
        raise SsdqError(fn, rc, last_error())
    return rc


def block_size(dtype: int) -> int:
    return lib().ssdq_block_size(dtype)


def type_size(dtype: int) -> int:
    return lib().ssdq_type_size(dtype)


def row_bytes(dtype: int, in_dim: int) -> int:
    return lib().ssdq_row_bytes(dtype, in_dim)


# ----------------------------------------------------------- torch helpers
def _ptr(t):
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def reserve_workspace(nbytes, stream=None):
    return check("ssdq_reserve_workspace", lib().ssdq_reserve_workspace(nbytes, _stream(stream)))


def release_workspaces():
    return check("ssdq_release_workspaces", lib().ssdq_release_workspaces())


def dequant(dtype, w, n_elements, out, stream=None):
    return check("ssdq_dequant_dev",
                 lib().ssdq_dequant_dev(dtype, _ptr(w), n_elements, _ptr(out), _stream(stream)))


def matvec(dtype, w, x, y, out_dim, in_dim, batch=1, stream=None, generic=False):
    f = lib().ssdq_matvec_generic_dev if generic else lib().ssdq_matvec_dev
    return check("ssdq_matvec_dev",
                 f(dtype, _ptr(w), _ptr(x), _ptr(y), out_dim, in_dim, batch, _stream(stream)))


def kv_slot_bytes(block_size, kv_dim):
    return lib().ssdq_kv_slot_bytes(block_size, kv_dim)


def kv_swap_out(k_codes, k_scales, v_codes, v_scales, block_ids, num_filled, n_blocks, block_size, kv_dim,
                n_pool_blocks, slots, stream=None):
    return check("ssdq_kv_swap_out_dev",
                 lib().ssdq_kv_swap_out_dev(_ptr(k_codes), _ptr(k_scales), _ptr(v_codes), _ptr(v_scales),
                                            _ptr(block_ids), _ptr(num_filled), n_blocks, block_size, kv_dim,
                                            n_pool_blocks, _ptr(slots), _stream(stream)))


def kv_swap_in(slots, block_ids, n_blocks, block_size, kv_dim, n_pool_blocks, k_codes, k_scales, v_codes,
               v_scales, num_filled, stream=None):
    return check("ssdq_kv_swap_in_dev",
                 lib().ssdq_kv_swap_in_dev(_ptr(slots), _ptr(block_ids), n_blocks, block_size, kv_dim,
                                           n_pool_blocks, _ptr(k_codes), _ptr(k_scales), _ptr(v_codes),
                                           _ptr(v_scales), _ptr(num_filled), _stream(stream)))


def qkv_rope(dtypes, ws, x, q, k, v, q_dim, kv_dim, n_embd, head_dim, position, theta, stream=None):
    (dq, dk, dv), (wq, wk, wv) = dtypes, ws
    return check("ssdq_qkv_rope_dev",
                 lib().ssdq_qkv_rope_dev(dq, _ptr(wq), dk, _ptr(wk), dv, _ptr(wv), _ptr(x), _ptr(q),
                                         _ptr(k), _ptr(v), q_dim, kv_dim, n_embd, head_dim, position,
                                         theta, _stream(stream)))


def swiglu(dtype, w_gate, w_up, x, h, n_ff, n_embd, stream=None):
    return check("ssdq_swiglu_dev",
                 lib().ssdq_swiglu_dev(dtype, _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(h), n_ff, n_embd,
                                       _stream(stream)))


def rmsnorm_matvec(dtype, w, x, norm_w, eps, y, out_dim, n_embd, stream=None):
    return check("ssdq_rmsnorm_matvec_dev",
                 lib().ssdq_rmsnorm_matvec_dev(dtype, _ptr(w), _ptr(x), _ptr(norm_w), eps, _ptr(y),
                                               out_dim, n_embd, _stream(stream)))


def rmsnorm(x, residual, weight, eps, hidden_out, out, n, stream=None):
    return check("ssdq_rmsnorm_dev",
                 lib().ssdq_rmsnorm_dev(_ptr(x), _ptr(residual), _ptr(weight), eps, _ptr(hidden_out),
                                        _ptr(out), n, _stream(stream)))


def gemm_q4k_bf16(w, x_bf16, y, M, N, K, stream=None):
    return check("ssdq_gemm_q4k_bf16_dev",
                 lib().ssdq_gemm_q4k_bf16_dev(_ptr(w), _ptr(x_bf16), _ptr(y), M, N, K,
                                              _stream(stream)))


def gemm_q4k_bf16_multi(ws, x_bf16, ys, M, ns, K, stream=None):
    """Y_i = X W_i^T for up to three Q4_K matrices sharing X, as one GEMM."""
    count = len(ws)
    if not (len(ys) == len(ns) == count):
        raise ValueError("ws, ys and ns must have the same length")
    warr = (_c.c_void_p * max(count, 1))(*[w.data_ptr() for w in ws])
    yarr = (_c.c_void_p * max(count, 1))(*[y.data_ptr() for y in ys])
    narr = (_c.c_size_t * max(count, 1))(*ns)
    return check("ssdq_gemm_q4k_bf16_multi_dev",
                 lib().ssdq_gemm_q4k_bf16_multi_dev(warr, narr, count, _ptr(x_bf16), yarr, M, K,
                                                    _stream(stream)))


def kv_quantize_rows(x, codes, scales, n_rows, row_len, stream=None):
    return check("ssdq_kv_quantize_rows_dev",
                 lib().ssdq_kv_quantize_rows_dev(_ptr(x), _ptr(codes), _ptr(scales), n_rows,
                                                 row_len, _stream(stream)))


def kv_dequantize_rows(codes, scales, out, n_rows, row_len, stream=None):
    return check("ssdq_kv_dequantize_rows_dev",
                 lib().ssdq_kv_dequantize_rows_dev(_ptr(codes), _ptr(scales), _ptr(out), n_rows,
                                                   row_len, _stream(stream)))


def paged_kv_append(k, v, slot_mapping, k_codes, k_scales, v_codes, v_scales, n_tokens, kv_dim,
                    stream=None):
    return check("ssdq_paged_kv_append_dev",
                 lib().ssdq_paged_kv_append_dev(_ptr(k), _ptr(v), _ptr(slot_mapping),
                                                _ptr(k_codes), _ptr(k_scales), _ptr(v_codes),
                                                _ptr(v_scales), n_tokens, kv_dim, _stream(stream)))


def paged_attention_int8(q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, out,
                         n_seq, n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq,
                         max_ctx, stream=None):
    return check("ssdq_paged_attention_int8_dev",
                 lib().ssdq_paged_attention_int8_dev(
                     _ptr(q), _ptr(k_codes), _ptr(k_scales), _ptr(v_codes), _ptr(v_scales),
                     _ptr(block_tables), _ptr(ctx_lens), _ptr(out), n_seq, n_head, n_head_kv,
                     head_dim, block_size, max_blocks_per_seq, max_ctx, _stream(stream)))


def paged_attention_int8_window(q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens,
                                window_starts, window_ends, out, n_seq, n_head, n_head_kv, head_dim, block_size,
                                max_blocks_per_seq, max_ctx, stream=None):
    """paged_attention_int8 over [window_starts[s], min(window_ends[s], ctx_lens[s])) per
    sequence (either tensor may be None)."""
    return check("ssdq_paged_attention_int8_window_dev",
                 lib().ssdq_paged_attention_int8_window_dev(
                     _ptr(q), _ptr(k_codes), _ptr(k_scales), _ptr(v_codes), _ptr(v_scales),
                     _ptr(block_tables), _ptr(ctx_lens), _ptr(window_starts), _ptr(window_ends), _ptr(out),
                     n_seq, n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq, max_ctx,
                     _stream(stream)))


def paged_attention_int8_noalloc(q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, out,
                                 n_seq, n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq,
                                 max_ctx, stream=None):
    """paged_attention_int8 with its partials in the library's static device
    scratch (16 MiB per GPU): allocates nothing; overlapping calls on one GPU race."""
    return check("ssdq_paged_attention_int8_noalloc_dev",
                 lib().ssdq_paged_attention_int8_noalloc_dev(
                     _ptr(q), _ptr(k_codes), _ptr(k_scales), _ptr(v_codes), _ptr(v_scales),
                     _ptr(block_tables), _ptr(ctx_lens), _ptr(out), n_seq, n_head, n_head_kv,
                     head_dim, block_size, max_blocks_per_seq, max_ctx, _stream(stream)))


def flash_attention_f32(q, k, v, out, n_head, n_head_kv, head_dim, seq_len, window_start,
                        window_end, stream=None):
    return check("ssdq_flash_attention_f32_dev",
                 lib().ssdq_flash_attention_f32_dev(_ptr(q), _ptr(k), _ptr(v), _ptr(out), n_head,
                                                    n_head_kv, head_dim, seq_len, window_start,
                                                    window_end, _stream(stream)))


class Context:
    """Host-pointer API with the MetalCompute contract (synchronous, copies in/out)."""

    def __init__(self, device: int = -1):
        h = ctypes.c_void_p()
        check("ssdq_ctx_create", lib().ssdq_ctx_create(device, ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib().ssdq_ctx_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def matvec_quantized(self, w_raw, x, out_dim, in_dim, dtype):
        """numpy in, numpy out: MetalCompute::matvec_quantized (compute.rs:157-191)."""
        import numpy as np
        w_raw = np.ascontiguousarray(w_raw, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(out_dim, np.float32)
        rc = lib().ssdq_matvec_quantized(self._h, w_raw.ctypes.data, w_raw.size, x.ctypes.data,
                                         x.size, out_dim, in_dim, dtype, y.ctypes.data)
        check("ssdq_matvec_quantized", rc)
        return y

    def dequantize_to_f32(self, data, dtype, n_elements):
        """dequantize_to_f32 (streamer.rs:93-125): bytes in, f32 numpy out."""
        import numpy as np
        data = np.ascontiguousarray(data, dtype=np.uint8)
        out = np.empty(n_elements, np.float32)
        rc = lib().ssdq_dequantize_to_f32(self._h, dtype, data.ctypes.data, data.size, n_elements,
                                          out.ctypes.data)
        check("ssdq_dequantize_to_f32", rc)
        return out

    def quantize_vectors_int8(self, data, dim):
        """quantize_vectors_int8 (block_swap.rs:36-60): (codes int8, scales f32)."""
        import numpy as np
        data = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        n_rows = data.size // dim
        codes = np.empty(n_rows * dim, np.int8)
        scales = np.empty(n_rows, np.float32)
        rc = lib().ssdq_quantize_vectors_int8(self._h, data.ctypes.data, n_rows, dim,
                                              codes.ctypes.data, scales.ctypes.data)
        check("ssdq_quantize_vectors_int8", rc)
        return codes, scales

    def dequantize_vectors_int8(self, codes, scales, dim):
        """dequantize_vectors_int8 (block_swap.rs:63-74)."""
        import numpy as np
        codes = np.ascontiguousarray(codes, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        out = np.empty(scales.size * dim, np.float32)
        rc = lib().ssdq_dequantize_vectors_int8(self._h, codes.ctypes.data, scales.ctypes.data,
                                                scales.size, dim, out.ctypes.data)
        check("ssdq_dequantize_vectors_int8", rc)
        return out

    def flash_attention_f32(self, q, k, v, n_head, n_head_kv, head_dim, seq_len, window_start,
                            window_end):
        import numpy as np
        q = np.ascontiguousarray(q, dtype=np.float32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        out = np.empty(n_head * head_dim, np.float32)
        rc = lib().ssdq_flash_attention_f32(self._h, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                            n_head, n_head_kv, head_dim, seq_len, window_start,
                                            window_end, out.ctypes.data)
        check("ssdq_flash_attention_f32", rc)
        return out


# ------------------------------------------------- resident weights + layer

class WeightStore:
    """GGUF tensors resident in HBM (ssdq_weights_*), uploaded once, found by
    name: the replacement of SsdStreamer::load_layer (src/ssd/streamer.rs:43-66),
    which dequantizes every tensor of a layer to f32 on each load."""

    def __init__(self, device: int = -1):
        h = _vp()
        check("ssdq_weights_create", lib().ssdq_weights_create(device, ctypes.byref(h)))
        self._h = h

    @property
    def handle(self):
        return self._h

    def put(self, name: str, dtype: int, dims, data) -> int:
        """dims as GGUF lists them (row length first); data: the raw bytes
        (bytes, or a numpy array whose buffer is the tensor's bytes).
        Returns the bytes uploaded."""
        import numpy as np
        buf = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray))
                                   else data).view(np.uint8).ravel()
        d = (_c.c_uint64 * len(dims))(*[int(v) for v in dims])
        check("ssdq_weights_put", lib().ssdq_weights_put(self._h, name.encode(), dtype, d, len(dims),
                                                         buf.ctypes.data, buf.nbytes))
        return buf.nbytes

    def load_layer(self, tensors, layer_idx: int) -> int:
        """Uploads the tensors of one layer (GgufFile::layer_tensors: names
        starting "blk.{layer_idx}.", gguf.rs:410-416) from (name, dtype, dims,
        data) tuples; returns the bytes made resident (CachedLayer::size_bytes)."""
        prefix = f"blk.{layer_idx}."
        return sum(self.put(name, dtype, dims, data) for name, dtype, dims, data in tensors
                   if name.startswith(prefix))

    def find(self, name: str):
        """(device address, dtype, dims, bytes) or None."""
        dt, nd, nb = _i(), _sz(), _sz()
        dims = (_c.c_uint64 * 4)()
        p = lib().ssdq_weights_find(self._h, name.encode(), ctypes.byref(dt), dims, ctypes.byref(nd),
                                    ctypes.byref(nb))
        if not p:
            return None
        return p, dt.value, tuple(dims[:nd.value]), nb.value

    def __len__(self):
        return lib().ssdq_weights_count(self._h)

    @property
    def nbytes(self) -> int:
        return lib().ssdq_weights_bytes(self._h)

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().ssdq_weights_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def layer_config(n_embd, n_head, n_head_kv, head_dim, n_ff, rope_theta, norm_eps=1e-5) -> LayerConfig:
    return LayerConfig(n_embd, n_head, n_head_kv, head_dim, n_ff, rope_theta, norm_eps)


def decode_layer_scratch(cfg: LayerConfig):
    """(bytes, {stage name: byte offset}) of ssdq_decode_layer_dev's scratch."""
    offs = (_sz * len(LAYER_STAGES))()
    n = lib().ssdq_decode_layer_scratch_bytes(ctypes.byref(cfg), offs)
    if n == 0:
        raise SsdqError("ssdq_decode_layer_scratch_bytes", -1, "bad layer config")
    return n, dict(zip(LAYER_STAGES, offs))


def decode_layer(store: WeightStore, layer: int, cfg: LayerConfig, hidden, position, k_codes, k_scales, v_codes,
                 v_scales, block_size, block_table, max_blocks_per_seq, slot_mapping, ctx_len, max_ctx,
                 scratch=None, stream=None):
    nbytes = scratch.numel() * scratch.element_size() if scratch is not None else 0
    return check("ssdq_decode_layer_dev",
                 lib().ssdq_decode_layer_dev(store.handle, layer, ctypes.byref(cfg), _ptr(hidden), position,
                                             _ptr(k_codes), _ptr(k_scales), _ptr(v_codes), _ptr(v_scales),
                                             block_size, _ptr(block_table), max_blocks_per_seq, _ptr(slot_mapping),
                                             _ptr(ctx_len), max_ctx, _ptr(scratch), nbytes, _stream(stream)))
