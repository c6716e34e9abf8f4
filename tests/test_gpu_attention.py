"""Decode attention parity: paged INT8 GQA (flash_attention.rs:70-139 over
paged_attention.rs:113-123 addressing and quantized_kv_cache.rs:49-53 dequant)
and the flat f32 MetalCompute::flash_attention_f32 surface (compute.rs:217-258).
Tolerance |gpu - ref| <= 1e-4 + 1e-3 |ref|."""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, assert_close, empty_dev, from_dev, to_dev
from ssdq import synth

pytestmark = pytest.mark.gpu


def paged_case(n_seq, n_head, n_kv, hd, bs, ctx_lens, mb, seed, quantize_on_gpu=False):
    g = np.random.default_rng(seed)
    rows = n_seq * mb * bs
    kv_dim = n_kv * hd
    tables = synth.block_tables(n_seq, mb, seed + 1)
    kf = g.standard_normal((rows, kv_dim), dtype=np.float32)
    vf = g.standard_normal((rows, kv_dim), dtype=np.float32)
    kc, ks = o.quantize_rows(kf, rows, kv_dim)
    vc, vs = o.quantize_rows(vf, rows, kv_dim)
    q = g.standard_normal((n_seq, n_head, hd), dtype=np.float32)
    return q, kc, ks, vc, vs, tables, np.asarray(ctx_lens, np.int32)


def run_paged(q, kc, ks, vc, vs, tables, ctx, n_seq, n_head, n_kv, hd, bs, mb):
    out = empty_dev(n_seq * n_head * hd, torch.float32)
    rc = ssdq.paged_attention_int8(to_dev(q), to_dev(kc), to_dev(ks), to_dev(vc), to_dev(vs),
                                   to_dev(tables), to_dev(ctx), out, n_seq, n_head, n_kv, hd, bs,
                                   mb, int(max(1, ctx.max())))
    return from_dev(out), rc


def test_paged_attention_config5_full_size():
    n_seq, n_head, n_kv, hd, bs, ctx = 8, 32, 8, 128, 16, 32768
    mb = ctx // bs
    announce("paged attention config5")
    q, kc, ks, vc, vs, tables, cl = paged_case(n_seq, n_head, n_kv, hd, bs, [ctx] * n_seq, mb, 500)
    got, rc = run_paged(q, kc, ks, vc, vs, tables, cl, n_seq, n_head, n_kv, hd, bs, mb)
    ref = o.paged_attention_int8(q, kc, ks, vc, vs, tables, cl, n_seq, n_head, n_kv, hd, bs, mb,
                                 threads=16)
    assert rc == 0
    assert_close(got, ref, "config5 attention")


CASES = [
    # n_seq, n_head, n_kv, hd, bs, ctx_lens
    (3, 32, 8, 128, 16, [0, 1, 15]),
    (4, 32, 8, 128, 16, [16, 17, 1000, 4095]),
    (2, 8, 8, 128, 16, [300, 77]),       # MHA (group 1)
    (2, 32, 4, 128, 16, [513, 64]),      # group 8
    (2, 16, 1, 64, 16, [999, 5]),        # MQA, head_dim 64
    (2, 8, 2, 256, 32, [700, 33]),       # head_dim 256, block 32
    (1, 48, 4, 128, 16, [257]),          # group 12 > 8 heads per pass
    (2, 4, 2, 128, 1, [50, 3]),          # block size 1
    (2, 48, 16, 64, 16, [200, 1500]),    # 16 KV heads (two 8-head workgroups), group 3
]


@pytest.mark.parametrize("n_seq,n_head,n_kv,hd,bs,ctx", CASES)
def test_paged_attention_cases(n_seq, n_head, n_kv, hd, bs, ctx):
    mb = max(1, -(-max(ctx) // bs)) + 1
    announce("paged attention", n_seq, n_head, n_kv, hd, bs, ctx)
    q, kc, ks, vc, vs, tables, cl = paged_case(n_seq, n_head, n_kv, hd, bs, ctx, mb, sum(ctx) + hd)
    got, rc = run_paged(q, kc, ks, vc, vs, tables, cl, n_seq, n_head, n_kv, hd, bs, mb)
    ref = o.paged_attention_int8(q, kc, ks, vc, vs, tables, cl, n_seq, n_head, n_kv, hd, bs, mb,
                                 threads=8)
    assert rc == 0
    assert_close(got, ref, "paged attention")
    empty = np.asarray(ctx) == 0
    assert np.all(got.reshape(n_seq, -1)[empty] == 0)


def test_paged_attention_rejects_bad_shapes():
    out = empty_dev(128, torch.float32)
    z = to_dev(np.zeros(1024, np.int32))
    with pytest.raises(ssdq.SsdqError):
        ssdq.paged_attention_int8(out, z, out, z, out, z, z, out, 1, 1, 1, 96, 16, 4, 64)
    with pytest.raises(ssdq.SsdqError):  # max_ctx beyond the block table
        ssdq.paged_attention_int8(out, z, out, z, out, z, z, out, 1, 1, 1, 128, 16, 4, 65)


FLAT = [
    # n_head, n_kv, hd, seq_len, window
    (32, 8, 128, 1, (0, 1)),
    (32, 8, 128, 2000, (0, 2000)),
    (8, 2, 64, 500, (100, 400)),
    (4, 4, 256, 129, (0, 10 ** 6)),
    (8, 8, 128, 10, (10, 20)),  # empty window -> zeros
]


@pytest.mark.parametrize("n_head,n_kv,hd,seq,window", FLAT)
def test_flash_attention_f32(n_head, n_kv, hd, seq, window):
    g = np.random.default_rng(seq + hd)
    q = g.standard_normal((n_head, hd), dtype=np.float32)
    k = g.standard_normal((seq, n_kv, hd), dtype=np.float32)
    v = g.standard_normal((seq, n_kv, hd), dtype=np.float32)
    out = empty_dev(n_head * hd, torch.float32)
    announce("flash f32", n_head, n_kv, hd, seq, window)
    ssdq.flash_attention_f32(to_dev(q), to_dev(k), to_dev(v), out, n_head, n_kv, hd, seq, *window)
    ref = o.flash_attention_f32(q, k, v, n_head, n_kv, hd, seq, *window)
    assert_close(from_dev(out), ref, "flash f32")


def test_flash_attention_host_twin():
    g = np.random.default_rng(3)
    n_head, n_kv, hd, seq = 32, 8, 128, 300
    q = g.standard_normal((n_head, hd), dtype=np.float32)
    k = g.standard_normal((seq, n_kv, hd), dtype=np.float32)
    v = g.standard_normal((seq, n_kv, hd), dtype=np.float32)
    announce("flash f32 host twin")
    with ssdq.Context() as ctx:
        got = ctx.flash_attention_f32(q, k, v, n_head, n_kv, hd, seq, 0, seq)
    ref = o.flash_attention_f32(q, k, v, n_head, n_kv, hd, seq, 0, seq)
    assert_close(got, ref, "host twin")


WINDOWS = [
    # n_seq, n_head, n_kv, hd, bs, ctx_lens, window starts, window ends
    # (the last sequence of the first case: start past its context -> zeros;
    # the second: an end past the context, an empty window, a window inside
    # one block, a start that is not block aligned)
    (4, 32, 8, 128, 16, [4096, 700, 33, 100], [1000, 0, 17, 200], [3000, 700, 10 ** 6, 300]),
    (4, 32, 8, 128, 16, [1000, 515, 64, 2048], [3, 300, 20, 1777], [5000, 300, 30, 2048]),
    (2, 8, 2, 256, 32, [900, 65], [64, 1], [800, 64]),              # head_dim 256, block 32
    (2, 16, 1, 64, 16, [999, 40], [500, 0], [999, 40]),             # MQA, head_dim 64
    (2, 4, 2, 128, 1, [50, 30], [10, 29], [49, 30]),                # block size 1
    (1, 32, 8, 128, 16, [32768], [32768 - 4096], [32768]),          # a 4k sliding window at 32k
]


@pytest.mark.parametrize("n_seq,n_head,n_kv,hd,bs,ctx,lo,hi", WINDOWS)
def test_paged_attention_window(n_seq, n_head, n_kv, hd, bs, ctx, lo, hi):
    """flash_attention_windowed (flash_attention.rs:146-227) over the paged INT8
    cache: positions [lo, min(hi, ctx)) per sequence, zeros when empty."""
    mb = max(1, -(-max(ctx) // bs))
    announce("paged attention window", n_seq, n_head, n_kv, hd, bs, ctx, lo, hi)
    q, kc, ks, vc, vs, tables, cl = paged_case(n_seq, n_head, n_kv, hd, bs, ctx, mb, sum(ctx) + 7 * hd)
    lo, hi = np.asarray(lo, np.int32), np.asarray(hi, np.int32)
    out = empty_dev(n_seq * n_head * hd, torch.float32)
    out.fill_(np.nan)
    rc = ssdq.paged_attention_int8_window(to_dev(q), to_dev(kc), to_dev(ks), to_dev(vc), to_dev(vs), to_dev(tables),
                                          to_dev(cl), to_dev(lo), to_dev(hi), out, n_seq, n_head, n_kv, hd, bs, mb,
                                          int(max(ctx)))
    assert rc == 0
    got = from_dev(out)
    ref = o.paged_attention_int8_window(q, kc, ks, vc, vs, tables, cl, lo, hi, n_seq, n_head, n_kv, hd, bs, mb,
                                        threads=8)
    assert_close(got, ref, "paged attention window")
    empty = np.minimum(hi, cl) <= lo
    assert np.all(got.reshape(n_seq, -1)[empty] == 0)
    # windows covering [0, ctx) reproduce the plain entry point bit for bit
    full, rc = run_paged(q, kc, ks, vc, vs, tables, cl, n_seq, n_head, n_kv, hd, bs, mb)
    assert rc == 0
    out.fill_(np.nan)
    rc = ssdq.paged_attention_int8_window(to_dev(q), to_dev(kc), to_dev(ks), to_dev(vc), to_dev(vs), to_dev(tables),
                                          to_dev(cl), None, None, out, n_seq, n_head, n_kv, hd, bs, mb, int(max(ctx)))
    assert rc == 0 and np.array_equal(from_dev(out).view(np.uint32), full.view(np.uint32))
