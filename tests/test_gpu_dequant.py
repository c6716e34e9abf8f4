"""Bit-exact device dequantization against the oracle (streamer.rs:128-220,
compute.rs:716-744) at the benchmark shapes, plus the f16 widening of every
scale bit pattern."""
import numpy as np
import pytest
import torch

import encoders as enc
import ssdq
import ssdq_oracle as o
from helpers import announce, empty_dev, first_bit_mismatch, from_dev, to_dev
from ssdq import synth

pytestmark = pytest.mark.gpu

SHAPES = [
    (ssdq.Q4_0, 4096, 4096),    # config 1
    (ssdq.Q4_0, 14336, 4096),   # north-star target shape
    (ssdq.Q8_0, 11008, 4096),   # config 2
    (ssdq.Q4_K, 14336, 4096),   # config 3 W_up
    (ssdq.Q6_K, 4096, 14336),   # config 3 W_down
]


@pytest.mark.parametrize("dtype,rows,cols", SHAPES)
def test_dequant_bit_exact_full_size(dtype, rows, cols):
    announce("dequant", ssdq.TYPE_NAMES[dtype], rows, cols)
    w = synth.quant_weights(dtype, rows, cols, synth.seed(3, dtype))
    n = rows * cols
    ref, rc = o.dequantize(dtype, w, n)
    out = empty_dev(n, torch.float32)
    assert ssdq.dequant(dtype, to_dev(w), n, out) == 0
    got = from_dev(out)
    assert first_bit_mismatch(got, ref) == -1


def test_f16_scale_widening_every_pattern():
    # One Q8_0 block per f16 bit pattern, codes +1 / -1: element = +-d exactly.
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blocks = np.zeros((65536, 34), np.uint8)
    blocks[:, 0] = pats & 0xFF
    blocks[:, 1] = pats >> 8
    blocks[:, 2] = 1
    blocks[:, 3] = 0xFF  # -1
    n = 65536 * 32
    announce("dequant f16 patterns")
    out = empty_dev(n, torch.float32)
    ssdq.dequant(ssdq.Q8_0, to_dev(blocks.ravel()), n, out)
    got = from_dev(out).reshape(65536, 32)
    ref, _ = o.dequantize(ssdq.Q8_0, blocks.ravel(), n)
    ref = ref.reshape(65536, 32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype", ssdq.QUANT_TYPES)
def test_dequant_encoder_fields(dtype):
    # every 6-bit scale / min at every Q4_K sub-block; every code at every position
    g = np.random.default_rng(dtype)
    blocks = []
    for i in range(64):
        if dtype == ssdq.Q4_K:
            s = (i + 7 * np.arange(8)) % 64
            m = (3 * i + 11 * np.arange(8) + 5) % 64
            blocks.append(enc.enc_q4_k(enc.f16_bits(g.uniform(.001, .01)), enc.f16_bits(g.uniform(.001, .01)),
                                       s, m, g.integers(0, 16, 256)))
        elif dtype == ssdq.Q6_K:
            blocks.append(enc.enc_q6_k(enc.f16_bits(g.uniform(.001, .01)),
                                       np.arange(-128, 128)[(i % 16) * 16:(i % 16 + 1) * 16],
                                       np.roll(np.arange(-32, 32).repeat(4), i)))
        elif dtype == ssdq.Q4_0:
            blocks.append(enc.enc_q4_0(enc.f16_bits(g.uniform(.002, .02)), np.roll(np.arange(-8, 8).repeat(2), i)))
        else:
            blocks.append(enc.enc_q8_0(enc.f16_bits(g.uniform(.002, .02)), np.arange(-128, 128)[(i % 8) * 32:(i % 8 + 1) * 32]))
    w = np.concatenate(blocks)
    n = 64 * ssdq.block_size(dtype)
    announce("dequant encoder", ssdq.TYPE_NAMES[dtype])
    out = empty_dev(n, torch.float32)
    ssdq.dequant(dtype, to_dev(w), n, out)
    ref, _ = o.dequantize(dtype, w, n)
    assert first_bit_mismatch(from_dev(out), ref) == -1


def test_dequant_tail_and_unsupported():
    w = synth.quant_weights(ssdq.Q4_K, 2, 256, 5)
    out = empty_dev(600, torch.float32)
    out.fill_(7.0)
    announce("dequant tail")
    assert ssdq.dequant(ssdq.Q4_K, to_dev(w), 600, out) == 0
    got = from_dev(out)
    ref, _ = o.dequantize(ssdq.Q4_K, w, 600)
    assert first_bit_mismatch(got, ref) == -1 and np.all(got[512:] == 0)
    out.fill_(7.0)
    assert ssdq.dequant(3, to_dev(w), 600, out) == ssdq.WARN_UNSUPPORTED_ZEROED
    assert np.all(from_dev(out) == 0)


@pytest.mark.parametrize("dtype", [ssdq.F32, ssdq.F16, ssdq.BF16])
def test_dequant_float_types_every_pattern(dtype):
    # F16 / BF16: all 65536 bit patterns; F32: random bits plus specials
    if dtype == ssdq.F32:
        g = np.random.default_rng(1)
        vals = np.concatenate([g.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32),
                               np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 1, 0x7FC00000],
                                        np.uint32)])
        raw = vals.view(np.uint8)
        n = vals.size
    else:
        raw = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8)
        n = 65536
    announce("dequant float type", dtype)
    out = empty_dev(n, torch.float32)
    assert ssdq.dequant(dtype, to_dev(raw), n, out) == 0
    got = from_dev(out)
    ref, rc = o.dequantize(dtype, raw, n)
    assert rc == 0
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype", ssdq.QUANT_TYPES)
def test_host_twin_dequantize_to_f32(dtype):
    # streamer.rs:93-125 contract: whole blocks present in data_len are decoded,
    # the rest of n_elements is zero
    rows, cols = 3, 512
    w = synth.quant_weights(dtype, rows, cols, dtype + 100)
    n = rows * cols
    bb = ssdq.type_size(dtype)
    announce("host twin dequantize_to_f32", ssdq.TYPE_NAMES[dtype])
    with ssdq.Context() as ctx:
        for data_len in (w.size, w.size - bb // 2, 2 * bb + 1, 0):
            got = ctx.dequantize_to_f32(w[:data_len], dtype, n)
            ref, _ = o.dequantize(dtype, w[:data_len], n)
            assert first_bit_mismatch(got, ref) == -1, data_len
        got = ctx.dequantize_to_f32(w, 3, n)  # Q4_1: unsupported -> zeros
        assert np.all(got == 0)
