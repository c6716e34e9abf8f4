"""Dequant-matvec parity for the reference's other matvec_quantized types:
Q2_K, Q3_K, Q5_K, Q8_K, IQ4_NL, IQ4_XS, F16, BF16 (matvec_*_cpu,
src/metal/compute.rs:796-1077, 2249-2285), through the C ABI.

Tolerance: |gpu - ref| <= 1e-4 + 1e-3 |ref| against the serial fp32 oracle,
with the exact-sum substitution of helpers.assert_close_attributed.  Covered:
full-size rows (K = 4096 and 14336, whose staged activations exceed 64 KB of
LDS), trailing partial blocks, batches 1-8, rows of 2-byte-aligned blocks
(Q3_K / IQ4_NL with an odd block count per row), the byte-addressed kernel,
misaligned weights, rows shorter than one block, and the host twin.
"""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, assert_close_attributed, empty_dev, from_dev, to_dev
from ssdq import synth

pytestmark = pytest.mark.gpu

TYPES = list(ssdq.MATVEC_EXTRA_TYPES)
# Signed 6-bit scales (IQ4_XS, Q3_K) make synthetic rows cancel heavily, so at
# K = 14336 the reference's serial fp32 sum itself strays past the tolerance on
# a few outputs; those are held to the same tolerance against the exact sum.
# The most seen is 3 of the 2000 outputs of IQ4_XS 1000 x 14336 batch 2, so
# this file allows 0.2% instead of the default 0.1%.
ILL = 2e-3


def run(dtype, w_dev, x, out_dim, in_dim, batch=1, generic=False):
    y = empty_dev(out_dim * batch, torch.float32)
    y.fill_(7.0)
    rc = ssdq.matvec(dtype, w_dev, to_dev(x), y, out_dim, in_dim, batch, generic=generic)
    return from_dev(y), rc


def reference(dtype, w, x, out_dim, in_dim, batch=1):
    x = np.asarray(x, np.float32).reshape(batch, -1)
    ys, ex = [], []
    for b in range(batch):
        ys.append(o.matvec(dtype, w, x[b], out_dim, in_dim, threads=16)[0])
        ex.append(o.matvec_exact(dtype, w, x[b], out_dim, in_dim))
    return np.concatenate(ys), np.concatenate(ex)


SHAPES = [
    # out_dim, in_dim, batch
    (4096, 4096, 1),
    (1000, 14336, 2),   # 448 groups: staged x over 64 KB
    (300, 4096 + 96, 3),  # trailing partial block ignored
    (50, 1000, 1),        # F16 / BF16: 1000 elements is no whole group -> byte-addressed kernel
    (77, 512, 8),
    (5, 256, 1),
]


@pytest.mark.parametrize("dtype", TYPES, ids=[ssdq.TYPE_NAMES[t] for t in TYPES])
@pytest.mark.parametrize("out_dim,in_dim,batch", SHAPES)
def test_ext_matvec(dtype, out_dim, in_dim, batch):
    w = synth.quant_weights(dtype, out_dim, in_dim, 1000 + dtype)
    x = synth.normal_f32((batch, in_dim), 2000 + in_dim)
    announce("matvec ext", ssdq.TYPE_NAMES[dtype], out_dim, in_dim, batch)
    y, rc = run(dtype, to_dev(w), x, out_dim, in_dim, batch)
    ref, exact = reference(dtype, w, x, out_dim, in_dim, batch)
    assert rc == 0
    n = assert_close_attributed(y, ref, exact, f"{ssdq.TYPE_NAMES[dtype]} {out_dim}x{in_dim} b{batch}",
                                max_ill_frac=ILL)
    print(f"{n} ill-conditioned outputs compared to the exact sum")


@pytest.mark.parametrize("dtype", TYPES, ids=[ssdq.TYPE_NAMES[t] for t in TYPES])
def test_ext_generic_kernel(dtype):
    w = synth.quant_weights(dtype, 300, 4096, 3000 + dtype)
    x = synth.normal_f32((3, 4096), 3001)
    announce("matvec ext generic", ssdq.TYPE_NAMES[dtype])
    y, rc = run(dtype, to_dev(w), x, 300, 4096, 3, generic=True)
    ref, exact = reference(dtype, w, x, 300, 4096, 3)
    assert rc == 0
    assert_close_attributed(y, ref, exact, "generic", max_ill_frac=ILL)


@pytest.mark.parametrize("dtype,in_dim", [(ssdq.Q3_K, 768), (ssdq.IQ4_NL, 96), (ssdq.Q3_K, 256 * 9),
                                          (ssdq.IQ4_NL, 32 * 45)])
def test_two_byte_aligned_blocks(dtype, in_dim):
    # an odd block count per row puts every other row's blocks at addresses = 2 mod 4
    w = synth.quant_weights(dtype, 129, in_dim, 4000 + in_dim)
    x = synth.normal_f32((2, in_dim), 4001)
    announce("matvec ext 2-byte aligned", ssdq.TYPE_NAMES[dtype], in_dim)
    y, rc = run(dtype, to_dev(w), x, 129, in_dim, 2)
    ref, exact = reference(dtype, w, x, 129, in_dim, 2)
    assert rc == 0
    assert_close_attributed(y, ref, exact, "2-byte aligned", max_ill_frac=ILL)


@pytest.mark.parametrize("dtype", TYPES, ids=[ssdq.TYPE_NAMES[t] for t in TYPES])
def test_misaligned_weights(dtype):
    w = synth.quant_weights(dtype, 64, 1024, 5000 + dtype)
    buf = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda")
    buf[2:2 + w.size] = to_dev(w)
    x = synth.normal_f32(1024, 5001)
    announce("matvec ext misaligned", ssdq.TYPE_NAMES[dtype])
    y, rc = run(dtype, buf[2:], x, 64, 1024)
    ref, exact = reference(dtype, w, x, 64, 1024)
    assert rc == 0
    assert_close_attributed(y, ref, exact, "misaligned", max_ill_frac=ILL)


def test_rows_shorter_than_a_block_are_zero():
    x = np.ones(100, np.float32)
    for dtype in (ssdq.Q5_K, ssdq.IQ4_XS, ssdq.Q2_K):
        announce("matvec ext short rows", ssdq.TYPE_NAMES[dtype])
        y, rc = run(dtype, to_dev(np.zeros(64, np.uint8)), x, 16, 100)
        assert rc == 0 and np.all(y == 0)


def test_known_answers_on_device():
    # compute.rs:2415-2433 (Q3_K -32), 2457-2493 (Q2_K 32), 2519-2535 (Q8_K 256),
    # 2727-2745 (IQ4_XS ~2.56) through the device path
    def f16(v):
        b = int(np.float16(v).view(np.uint16))
        return b & 0xFF, b >> 8

    q3 = np.zeros(110, np.uint8)
    q3[108], q3[109] = f16(0.5)
    q3[96] = 1
    q2 = np.zeros(84, np.uint8)
    q2[0], q2[1] = f16(1.0)
    q2[4] = 2
    q2[20:24] = 0x55
    q8 = np.zeros(292, np.uint8)
    q8[0:4] = np.array([1.0], np.float32).view(np.uint8)
    q8[4:260] = 1
    xs = np.zeros(148, np.uint8)
    xs[0], xs[1] = f16(0.01)
    xs[2] = xs[3] = 0xAA
    xs[4:20:2] = 0x11
    xs[20:148] = 0x88
    announce("matvec ext KATs")
    for dtype, blk, want, tol in ((ssdq.Q3_K, q3, -32.0, 1e-3), (ssdq.Q2_K, q2, 32.0, 1e-3),
                                  (ssdq.Q8_K, q8, 256.0, 1e-3), (ssdq.IQ4_XS, xs, 2.56, 0.5)):
        y, rc = run(dtype, to_dev(blk), np.ones(256, np.float32), 1, 256)
        assert rc == 0 and abs(y[0] - want) < tol, (dtype, y[0])


def test_host_twin_new_types():
    with ssdq.Context() as ctx:
        for dtype in (ssdq.Q5_K, ssdq.IQ4_NL, ssdq.BF16):
            w = synth.quant_weights(dtype, 512, 2048, 6000 + dtype)
            x = synth.normal_f32(2048, 6001)
            announce("matvec ext host twin", ssdq.TYPE_NAMES[dtype])
            y = ctx.matvec_quantized(w, x, 512, 2048, dtype)
            ref, exact = reference(dtype, w, x, 512, 2048)
            assert_close_attributed(y, ref, exact, "host twin", max_ill_frac=ILL)
        # F32 stays unsupported (compute.rs:672-675)
        y = ctx.matvec_quantized(np.zeros(256, np.uint8), np.ones(8, np.float32), 8, 8, ssdq.F32)
        assert np.all(y == 0)


@pytest.mark.parametrize("dtype", [ssdq.Q5_K, ssdq.Q2_K, ssdq.Q3_K, ssdq.Q8_K], ids=["Q5_K", "Q2_K", "Q3_K", "Q8_K"])
@pytest.mark.parametrize("out_dim,in_dim", [(14336, 4096), (4096, 14336), (77, 768), (130, 256 * 5)])
def test_batch1_digit_kernel(dtype, out_dim, in_dim):
    # batch 1 with aligned weights (Q5_K: 16 bytes, Q2_K / Q3_K / Q8_K: 4) runs the
    # digit-plane kernel (K-sliced past 128 units per row; Q3_K rows of an odd
    # block count start 2 bytes off a dword); the byte-addressed float kernel is
    # the cross-check
    w = synth.quant_weights(dtype, out_dim, in_dim, 7000 + in_dim + dtype)
    x = synth.normal_f32(in_dim, 7001)
    name = ssdq.TYPE_NAMES[dtype]
    announce("matvec digit", name, out_dim, in_dim)
    y, rc = run(dtype, to_dev(w), x, out_dim, in_dim)
    assert rc == 0
    sel = np.arange(out_dim) if out_dim <= 4096 else np.r_[0:2048, out_dim - 2048:out_dim]
    rows = synth.BLOCK[dtype][1] * (in_dim // 256)
    wsel = w.reshape(out_dim, rows)[sel].ravel()
    ref, exact = reference(dtype, wsel, x, sel.size, in_dim)
    assert_close_attributed(y[sel], ref, exact, f"{name} digit {out_dim}x{in_dim}", max_ill_frac=ILL)
    yg, rcg = run(dtype, to_dev(w), x, out_dim, in_dim, generic=True)
    assert rcg == 0
    assert_close_attributed(y[sel], yg[sel], exact, "digit vs float kernel", max_ill_frac=ILL)
