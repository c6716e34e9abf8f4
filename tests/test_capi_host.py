"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and its pure-host helpers agree with the GGUF type table."""
import ctypes
import os
import re

import pytest

import ssdq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ssdq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ssdq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("ssdq_matvec_dev", "ssdq_matvec_quantized", "ssdq_dequant_dev",
                     "ssdq_gemm_q4k_bf16_dev", "ssdq_kv_quantize_rows_dev",
                     "ssdq_kv_dequantize_rows_dev", "ssdq_paged_kv_append_dev",
                     "ssdq_paged_attention_int8_dev", "ssdq_flash_attention_f32_dev",
                     "ssdq_flash_attention_f32", "ssdq_ctx_create", "ssdq_ctx_destroy"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ssdq.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers all of them with signatures
    assert set(declared_functions()) <= set(ssdq.SIGNATURES)


def test_type_helpers():
    assert ssdq.lib().ssdq_abi_version() == 1
    for dt, bs, ts in ((ssdq.Q4_0, 32, 18), (ssdq.Q8_0, 32, 34), (ssdq.Q4_K, 256, 144),
                       (ssdq.Q6_K, 256, 210)):
        assert ssdq.block_size(dt) == bs and ssdq.type_size(dt) == ts
        assert ssdq.row_bytes(dt, 4096) == 4096 // bs * ts
        assert ssdq.row_bytes(dt, 4096 + bs - 1) == 4096 // bs * ts  # partial block ignored
    assert ssdq.block_size(99) == 0 and ssdq.row_bytes(99, 4096) == 0
    # the other matvec types agree with the oracle's table (Q3_K: 110-byte blocks)
    import ssdq_oracle as o
    for dt in ssdq.MATVEC_EXTRA_TYPES:
        assert (ssdq.block_size(dt), ssdq.type_size(dt)) == (o.block_size(dt), o.type_size(dt)), dt
    assert ssdq.type_size(ssdq.Q3_K) == 110


def test_null_arguments_are_rejected_without_a_device():
    lib = ssdq.lib()
    # zero-sized calls are no-ops; NULL outputs are argument errors, checked before any HIP call
    assert lib.ssdq_matvec_dev(ssdq.Q4_K, None, None, None, 0, 4096, 1, None) == 0
    assert lib.ssdq_matvec_dev(ssdq.Q4_K, None, None, None, 16, 4096, 1, None) == -1
    assert "NULL" in ssdq.last_error()
    assert lib.ssdq_kv_quantize_rows_dev(None, None, None, 4, 16, None) == -1
    assert lib.ssdq_paged_attention_int8_dev(*([None] * 8), 1, 8, 2, 100, 16, 4, 64, None) == -1
    assert lib.ssdq_gemm_q4k_bf16_dev(None, None, None, 4, 4, 256, None) == -1


def test_ctx_create_reports_missing_device():
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    h = ctypes.c_void_p()
    rc = ssdq.lib().ssdq_ctx_create(-1, ctypes.byref(h))
    assert rc == -4 and not h.value  # SSDQ_ERR_NO_DEVICE: callers keep their CPU path


def test_cpp_host_mirror_header_compiles():
    """The C++ mirror header is self-contained C++17 over include/ssdq.h."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    hdr = os.path.join(root, "ssd-llm_amd", "host", "ssdq_compute.hpp")
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-x", "c++", hdr],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_noalloc_attention_rejects_oversized_partials_before_launch():
    # 4096 sequences x 64 heads need >= 136 MB of split partials against the
    # 16 MiB static scratch: rejected from the arguments alone, before any HIP
    # launch (the dummy, never-dereferenced pointers are 256-aligned)
    lib = ssdq.lib()
    p = ctypes.c_void_p(256)
    rc = lib.ssdq_paged_attention_int8_noalloc_dev(p, p, p, p, p, p, p, p, 4096, 64, 8, 128, 16, 64, 1024, None)
    assert rc == -1
    assert "scratch" in ssdq.last_error()


def test_weight_store_and_layer_layout_on_the_host():
    lib = ssdq.lib()
    try:
        import torch
        gpu = torch.cuda.is_available()
    except ImportError:
        gpu = False
    if not gpu:
        h = ctypes.c_void_p()
        assert lib.ssdq_weights_create(-1, ctypes.byref(h)) == -4 and not h.value
    # NULL store / hidden state: argument errors before any HIP call
    cfg = ssdq.layer_config(4096, 32, 8, 128, 14336, 500000.0)
    assert lib.ssdq_decode_layer_dev(None, 0, ctypes.byref(cfg), None, 0, *([None] * 4), 16, None, 1, None, None,
                                     16, None, 0, None) == -1
    assert lib.ssdq_weights_find(None, b"blk.0.attn_q.weight", None, None, None, None) is None
    assert lib.ssdq_weights_count(None) == 0 and lib.ssdq_weights_device(None) == -1
    # the scratch layout: one 256-byte aligned region per step, in order
    n, offs = ssdq.decode_layer_scratch(cfg)
    sizes = dict(attn_in=4096, q=4096, k=1024, v=1024, attn=4096, attn_out=4096, ffn_in=4096, ffn_h=14336,
                 ffn_gate=14336, ffn_up=14336, ffn_out=4096, norm_w=8192, hidden_mid=4096)
    at = 0
    for name in ssdq.LAYER_STAGES:
        assert offs[name] == at and at % 256 == 0
        at += -(-4 * sizes[name] // 256) * 256
    assert n == at
    # head sizes outside the attention kernels', and n_head not a multiple of n_head_kv
    for bad in (ssdq.layer_config(4096, 32, 8, 96, 14336, 1e4), ssdq.layer_config(4096, 30, 8, 128, 14336, 1e4)):
        assert lib.ssdq_decode_layer_scratch_bytes(ctypes.byref(bad), None) == 0
