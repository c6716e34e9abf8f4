"""Bit-exact INT8 KV quantization (block_swap.rs:36-74, quantized_kv_cache.rs:23-53)
and the paged quantize-on-append."""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, empty_dev, from_dev, to_dev
from ssdq import synth

pytestmark = pytest.mark.gpu


def gpu_quantize(x, n_rows, dim):
    c = empty_dev(n_rows * dim, torch.int8)
    s = empty_dev(n_rows, torch.float32)
    assert ssdq.kv_quantize_rows(to_dev(x), c, s, n_rows, dim) == 0
    return from_dev(c), from_dev(s)


def test_quantize_config5_full_size():
    # 8 sequences x 32768 tokens x {K, V} rows of kv_dim 1024
    n_rows, dim = 8 * 32768 * 2, 1024
    announce("kv quantize config5", n_rows, dim)
    x = synth.normal_f32(n_rows * dim, synth.seed(5, 0))
    c, s = gpu_quantize(x, n_rows, dim)
    rc, rs = o.quantize_rows(x, n_rows, dim)
    assert np.array_equal(c, rc)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def edge_rows(dim):
    g = np.random.default_rng(5)
    rows = g.standard_normal((16, dim)).astype(np.float32)
    rows[0] = 0                                    # -> scale 0, codes 0
    rows[1, :dim // 2] = np.nan                    # NaN ignored by absmax, coded 0
    rows[2, 3] = np.inf                            # scale inf, finite -> 0, inf -> NaN -> 0
    rows[3] *= np.float32(1e-42)                   # subnormal absmax, 127/absmax overflows
    rows[4] = np.float32(127.0) * (np.arange(dim) % 7 - 3) / 3  # exact ties after scaling
    rows[5] = -rows[6]                             # symmetry
    rows[7, 0] = np.float32(3e38)                  # huge
    rows[8] = np.float32(-0.0)                     # all negative zeros
    rows[9, :] = np.nan                            # all NaN -> absmax 0
    rows[10] = np.linspace(-1, 1, dim).astype(np.float32)
    rows[11] = np.float32(0.5) + np.arange(dim, dtype=np.float32)
    return rows


@pytest.mark.parametrize("dim", [1024, 128, 1000, 7, 4100, 2048])
def test_quantize_edge_rows(dim):
    rows = edge_rows(dim)
    announce("kv quantize edges", dim)
    c, s = gpu_quantize(rows, rows.shape[0], dim)
    rc, rs = o.quantize_rows(rows, rows.shape[0], dim)
    assert np.array_equal(c, rc)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_quantize_unaligned_input():
    dim, n = 1024, 64
    x = synth.normal_f32(n * dim + 1, 6)
    xd = to_dev(x)
    c = empty_dev(n * dim, torch.int8)
    s = empty_dev(n, torch.float32)
    announce("kv quantize unaligned")
    ssdq.kv_quantize_rows(xd[1:], c, s, n, dim)
    rc, rs = o.quantize_rows(x[1:], n, dim)
    assert np.array_equal(from_dev(c), rc) and np.array_equal(from_dev(s), rs)


def test_dequantize_bit_exact():
    n, dim = 4096, 1024
    x = synth.normal_f32(n * dim, 7)
    rc, rs = o.quantize_rows(x, n, dim)
    out = empty_dev(n * dim, torch.float32)
    announce("kv dequantize")
    assert ssdq.kv_dequantize_rows(to_dev(rc), to_dev(rs), out, n, dim) == 0
    ref = o.dequantize_rows(rc, rs, n, dim)
    assert np.array_equal(from_dev(out).view(np.uint32), ref.view(np.uint32))


def test_paged_append_places_quantized_rows():
    n_seq, bs, mb, kv_dim = 4, 16, 40, 1024
    ctx = [1, 16, 17, 600]
    tables = synth.block_tables(n_seq, mb, 8)
    slots = synth.slot_mapping(tables, ctx, bs)
    slots[5] = -1  # a padding token is skipped
    n_tok = slots.size
    k = synth.normal_f32((n_tok, kv_dim), 9)
    v = synth.normal_f32((n_tok, kv_dim), 10)
    pool_rows = n_seq * mb * bs
    kc = torch.full((pool_rows * kv_dim,), 99, dtype=torch.int8, device="cuda")
    vc = torch.full((pool_rows * kv_dim,), 99, dtype=torch.int8, device="cuda")
    ks = torch.full((pool_rows,), -1.0, dtype=torch.float32, device="cuda")
    vs = torch.full((pool_rows,), -1.0, dtype=torch.float32, device="cuda")
    announce("paged append")
    assert ssdq.paged_kv_append(to_dev(k), to_dev(v), to_dev(slots), kc, ks, vc, vs, n_tok, kv_dim) == 0
    kc, vc, ks, vs = from_dev(kc).reshape(pool_rows, kv_dim), from_dev(vc).reshape(pool_rows, kv_dim), from_dev(ks), from_dev(vs)
    rkc, rks = o.quantize_rows(k, n_tok, kv_dim)
    rvc, rvs = o.quantize_rows(v, n_tok, kv_dim)
    rkc, rvc = rkc.reshape(n_tok, kv_dim), rvc.reshape(n_tok, kv_dim)
    live = slots >= 0
    assert np.array_equal(kc[slots[live]], rkc[live]) and np.array_equal(vc[slots[live]], rvc[live])
    assert np.array_equal(ks[slots[live]], rks[live]) and np.array_equal(vs[slots[live]], rvs[live])
    untouched = np.setdiff1d(np.arange(pool_rows), slots[live])
    assert np.all(kc[untouched] == 99) and np.all(ks[untouched] == -1.0)


def test_host_twin_int8_vectors():
    # quantize_vectors_int8 / dequantize_vectors_int8 (block_swap.rs:36-74)
    dim = 128
    x = np.random.default_rng(9).standard_normal((40, dim), dtype=np.float32)
    x[3] = 0.0          # zero row -> scale 0, codes 0
    x[7, 5] = 1e30      # one huge element
    announce("host twin int8 vectors")
    with ssdq.Context() as ctx:
        codes, scales = ctx.quantize_vectors_int8(x, dim)
        back = ctx.dequantize_vectors_int8(codes, scales, dim)
    rc, rs = o.quantize_rows(x, 40, dim)
    assert np.array_equal(codes, rc)
    assert np.array_equal(scales.view(np.uint32), rs.view(np.uint32))
    ref = o.dequantize_rows(rc, rs, 40, dim)
    assert np.array_equal(back.view(np.uint32), ref.view(np.uint32))
    assert scales[3] == 0 and np.all(codes[3 * dim:4 * dim] == 0)
