"""Pins the oracle's restatements of the reference's other matvec types
(Q2_K, Q3_K, Q5_K, Q8_K, IQ4_NL, IQ4_XS, F16, BF16; compute.rs:796-1077,
2249-2285) before they are trusted as the checker:
  * every known-answer test the reference holds for them (compute.rs:2383-2746);
  * encoder round trips: tests/encoders.py packs chosen codes and scales, and
    the oracle's matvec against unit vectors must return exactly the element
    values those fields define, for every code at every position;
  * two-path agreement: the matvec equals the serial fp32 sum, in the
    reference's order, of the encoder's elements times x (Q5_K sums pairs);
  * the exact (double) path agrees with the encoder's elements, and the fp32
    matvec stays within the serial-summation error bound of it.
"""
import numpy as np
import pytest

import encoders as enc
import ssdq_oracle as o

F16, Q2_K, Q3_K, Q5_K, Q8_K, IQ4_NL, IQ4_XS, BF16 = 1, 10, 11, 13, 15, 20, 23, 30


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _f16(v):
    return int(enc.f16_bits(v))


def test_type_table_matches_gguf():
    # src/model/gguf.rs:87-135, except Q3_K: gguf.rs:127 computes 256/8*3 + ... = 174
    # bytes, but matvec_q3_k_cpu (compute.rs:798) and the GGUF format read 110-byte
    # blocks (32 hmask + 64 qs + 12 scales + 2 d); the matvec's layout is the one kept
    want = {Q2_K: (256, 84), Q3_K: (256, 110), Q5_K: (256, 176), Q8_K: (256, 292),
            IQ4_NL: (32, 18), IQ4_XS: (256, 148), F16: (1, 2), BF16: (1, 2), 16: (256, 66),
            17: (256, 74), 18: (256, 98), 21: (256, 110)}
    for t, v in want.items():
        assert (o.block_size(t), o.type_size(t)) == v, t


# ---------------------------------------------- reference known answers
def _kat(dtype, blk, x, n_rows=1):
    y, rc = o.matvec(dtype, np.asarray(blk, np.uint8), np.asarray(x, np.float32), n_rows, len(x))
    assert rc == 0
    return y


def test_q3_k_known_answers():
    # compute.rs:2383-2397 (zero scales -> 0) and 2415-2433 (sc[0] = 1, d = 0.5 -> -32)
    blk = np.zeros(110, np.uint8)
    blk[108], blk[109] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
    assert abs(_kat(Q3_K, blk, np.ones(256))[0]) < 1e-5
    blk = np.zeros(110, np.uint8)
    blk[108], blk[109] = _f16(0.5) & 0xFF, _f16(0.5) >> 8
    blk[96] = 0x01
    assert abs(_kat(Q3_K, blk, np.ones(256))[0] - (-32.0)) < 1e-3


def test_q5_k_known_answers():
    # compute.rs:2399-2413 and 2435-2455
    blk = np.zeros(176, np.uint8)
    blk[0], blk[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
    assert abs(_kat(Q5_K, blk, np.ones(256))[0]) < 1e-5
    blk[4] = 0x01
    blk[48:64] = 0x11
    assert abs(_kat(Q5_K, blk, np.ones(256))[0] - 32.0) < 1e-3


def test_q2_k_known_answers():
    # compute.rs:2457-2470, 2472-2493, 2495-2517
    blk = np.zeros(84, np.uint8)
    blk[0], blk[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
    assert abs(_kat(Q2_K, blk, np.ones(256))[0]) < 1e-5
    blk[4] = 0x02
    blk[20:24] = 0x55
    assert abs(_kat(Q2_K, blk, np.ones(256))[0] - 32.0) < 1e-3
    blk = np.zeros(84, np.uint8)
    blk[0], blk[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
    blk[2], blk[3] = _f16(0.5) & 0xFF, _f16(0.5) >> 8
    blk[4] = 0x20
    assert abs(_kat(Q2_K, blk, np.ones(256))[0] - (-16.0)) < 1e-3


def test_q8_k_known_answers():
    # compute.rs:2519-2535 and 2537-2555
    blk = np.zeros(292, np.uint8)
    blk[0:4] = np.array([1.0], np.float32).view(np.uint8)
    blk[4:260] = 1
    assert abs(_kat(Q8_K, blk, np.ones(256))[0] - 256.0) < 1e-3
    blk[0:4] = np.array([0.5], np.float32).view(np.uint8)
    blk[4:260] = 0xFE
    assert abs(_kat(Q8_K, blk, np.ones(256))[0] - (-256.0)) < 1e-3


def test_iq4_nl_known_answers():
    # compute.rs:2564-2585, 2587-2608, 2610-2640, 2712-2725
    blk = np.zeros(18, np.uint8)
    blk[0], blk[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
    assert abs(_kat(IQ4_NL, blk, np.ones(32))[0] - (-127.0 * 32)) < 1.0
    blk = np.zeros(18, np.uint8)
    blk[0], blk[1] = _f16(0.5) & 0xFF, _f16(0.5) >> 8
    blk[2] = 0xF8
    x = np.zeros(32, np.float32)
    x[0] = x[1] = 1.0
    assert abs(_kat(IQ4_NL, blk, x)[0] - 0.5 * (1.0 + 113.0)) < 0.5
    data = np.zeros(36, np.uint8)
    data[0], data[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
    data[2:18] = 0x88
    data[18], data[19] = _f16(2.0) & 0xFF, _f16(2.0) >> 8
    data[20:36] = 0x88
    y = _kat(IQ4_NL, data, np.ones(32), n_rows=2)
    assert abs(y[0] - 32.0) < 1.0 and abs(y[1] - 64.0) < 1.0
    # code book end points and zero crossing (compute.rs:2704-2710)
    one = np.zeros(18, np.uint8)
    one[0], one[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
    for idx, val in ((0, -127), (15, 113), (8, 1)):
        one[2] = idx
        x = np.zeros(32, np.float32)
        x[0] = 1.0
        assert _kat(IQ4_NL, one, x)[0] == val


def test_iq4_xs_known_answers():
    # compute.rs:2642-2673, 2675-2702, 2727-2745
    blk = np.zeros(148, np.uint8)
    blk[0], blk[1] = _f16(1.0) & 0xFF, _f16(1.0) >> 8
    blk[20:148] = 0x88
    assert abs(_kat(IQ4_XS, blk, np.ones(256))[0] - (-32.0 * 256)) < 10.0
    blk = np.zeros(148, np.uint8)
    blk[0], blk[1] = _f16(0.01) & 0xFF, _f16(0.01) >> 8
    blk[2] = blk[3] = 0xAA
    blk[4:20:2] = 0x11
    blk[20:148] = 0x88
    assert abs(_kat(IQ4_XS, blk, np.ones(256))[0] - 2.56) < 0.5


def test_f16_bf16_known_answers():
    # matvec_f16_cpu / matvec_bf16_cpu (compute.rs:2256-2285): plain products
    w = np.array([1.0, -2.0, 0.5, 4.0], np.float16).view(np.uint8)
    assert np.array_equal(_kat(F16, w, [3.0, 1.0], n_rows=2), np.array([1.0, 5.5], np.float32))
    wb = (np.array([1.0, -2.0, 0.5, 4.0], np.float32).view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(_kat(BF16, wb.view(np.uint8), [3.0, 1.0], n_rows=2),
                          np.array([1.0, 5.5], np.float32))


def test_f32_stays_unsupported():
    # F32 is not in matvec_quantized_cpu's match (compute.rs:655-676): zeros
    y, rc = o.matvec(0, np.ones(64, np.float32).view(np.uint8), np.ones(8, np.float32), 2, 8)
    assert rc == 1 and np.all(y == 0)


# ------------------------------------------------- encoder round trips
def _cases(dtype, n, g):
    """n blocks of one format with every code at every position; returns
    (block bytes, expected elements)."""
    blocks, want = [], []
    for i in range(n):
        if dtype == Q2_K:
            d, dm = _f16(g.uniform(0.001, 0.01)), _f16(g.uniform(0.001, 0.01))
            s, m = (i + np.arange(16)) % 16, (3 * i + 5 * np.arange(16)) % 16
            q = np.roll(np.arange(256) % 4, i)
            blocks.append(enc.enc_q2_k(d, dm, s, m, q))
            want.append(enc.dec_expect_q2_k(d, dm, s, m, q))
        elif dtype == Q3_K:
            d = _f16(g.uniform(0.001, 0.01))
            sv = ((i * 16 + np.arange(16)) % 64) - 32
            q = np.roll(np.arange(256) % 8 - 4, 3 * i)
            blocks.append(enc.enc_q3_k(d, sv, q))
            want.append(enc.dec_expect_q3_k(d, sv, q))
        elif dtype == Q5_K:
            d, dm = _f16(g.uniform(0.001, 0.01)), _f16(g.uniform(0.001, 0.01))
            s, m = (i + 7 * np.arange(8)) % 64, (3 * i + 11 * np.arange(8) + 5) % 64
            q = np.roll(np.arange(256) % 32, 5 * i)
            blocks.append(enc.enc_q5_k(d, dm, s, m, q))
            want.append(enc.dec_expect_q5_k(d, dm, s, m, q))
        elif dtype == Q8_K:
            d = np.float32(g.uniform(0.001, 0.01))
            q = np.roll(np.arange(-128, 128), 17 * i)
            blocks.append(enc.enc_q8_k(d, q))
            want.append(enc.dec_expect_q8_k(d, q))
        elif dtype == IQ4_NL:
            d = _f16(g.uniform(0.002, 0.02))
            idx = np.roll(np.arange(32) % 16, i)
            blocks.append(enc.enc_iq4_nl(d, idx))
            want.append(enc.dec_expect_iq4_nl(d, idx))
        elif dtype == IQ4_XS:
            d = _f16(g.uniform(0.0001, 0.001))
            s6 = (8 * i + np.arange(8)) % 64
            idx = np.roll(np.arange(256) % 16, 3 * i)
            blocks.append(enc.enc_iq4_xs(d, s6, idx))
            want.append(enc.dec_expect_iq4_xs(d, s6, idx))
    return np.stack(blocks), np.stack(want)


EXT = [Q2_K, Q3_K, Q5_K, Q8_K, IQ4_NL, IQ4_XS]
N_CASES = {Q2_K: 16, Q3_K: 4, Q5_K: 16, Q8_K: 16, IQ4_NL: 16, IQ4_XS: 8}


def _elements_via_unit_vectors(dtype, blocks):
    n, bb = blocks.shape
    k = o.block_size(dtype)
    out = np.empty((n, k), np.float32)
    for j in range(k):
        x = np.zeros(k, np.float32)
        x[j] = 1.0
        y, rc = o.matvec(dtype, blocks.reshape(-1), x, n, k)
        assert rc == 0
        out[:, j] = y
    return out


@pytest.mark.parametrize("dtype", EXT)
def test_layout_round_trip(dtype):
    blocks, want = _cases(dtype, N_CASES[dtype], np.random.default_rng(dtype))
    got = _elements_via_unit_vectors(dtype, blocks)
    # the serial sum 0 + e*1 turns a -0 element into +0; every other bit must match
    assert np.array_equal(_bits(got + np.float32(0)), _bits(want + np.float32(0)))


@pytest.mark.parametrize("dtype", EXT)
def test_exact_path_elements_match_encoder(dtype):
    # the decoder behind the exact (double) sums reproduces the encoder's fields
    blocks, want = _cases(dtype, N_CASES[dtype], np.random.default_rng(dtype + 100))
    k = o.block_size(dtype)
    e, rc = o.matvec_elements(dtype, blocks.reshape(-1), len(blocks), k)
    assert rc == 0 and np.array_equal(_bits(e), _bits(want))
    x = np.random.default_rng(5).standard_normal(k).astype(np.float32)
    ex = o.matvec_exact(dtype, blocks.reshape(-1), x, len(blocks), k)
    assert np.allclose(ex, (want.astype(np.float64) * x).sum(1), rtol=1e-12, atol=1e-12)


def _serial_sum(terms):
    s = np.zeros(terms.shape[0], np.float32)
    for i in range(terms.shape[1]):
        s = (s + terms[:, i]).astype(np.float32)
    return s


@pytest.mark.parametrize("dtype", EXT)
def test_matvec_equals_serial_sum_in_reference_order(dtype):
    g = np.random.default_rng(dtype + 200)
    blocks, want = _cases(dtype, N_CASES[dtype], g)
    k = o.block_size(dtype)
    x = g.standard_normal(k).astype(np.float32)
    y, rc = o.matvec(dtype, blocks.reshape(-1), x, len(blocks), k)
    prod = (want * x[None, :]).astype(np.float32)
    if dtype == Q5_K:  # sum += v0 * x[i0] + v1 * x[i1]  (compute.rs:896)
        prod = (prod[:, 0::2] + prod[:, 1::2]).astype(np.float32)
    assert rc == 0 and np.array_equal(_bits(y), _bits(_serial_sum(prod)))


def test_float_types_serial_sum():
    g = np.random.default_rng(9)
    w = (g.standard_normal((5, 300)) * 0.1).astype(np.float32)
    x = g.standard_normal(300).astype(np.float32)
    wh = w.astype(np.float16)
    y, _ = o.matvec(F16, wh.view(np.uint8).reshape(-1), x, 5, 300)
    assert np.array_equal(_bits(y), _bits(_serial_sum((wh.astype(np.float32) * x).astype(np.float32))))
    wb = (w.view(np.uint32) >> 16).astype(np.uint16)
    y, _ = o.matvec(BF16, wb.view(np.uint8).reshape(-1), x, 5, 300)
    wbf = (wb.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(_bits(y), _bits(_serial_sum((wbf * x).astype(np.float32))))


@pytest.mark.parametrize("dtype", EXT + [F16, BF16, 16, 17, 18, 21])
def test_matvec_within_fp32_bound_of_exact(dtype):
    from ssdq import synth
    out_dim, in_dim = 32, 4096
    w = synth.quant_weights(dtype, out_dim, in_dim, 21)
    x = synth.normal_f32(in_dim, 22)
    y, rc = o.matvec(dtype, w, x, out_dim, in_dim)
    ex = o.matvec_exact(dtype, w, x, out_dim, in_dim)
    e, _ = o.matvec_elements(dtype, w, out_dim, in_dim)
    absum = (np.abs(e.astype(np.float64)) * np.abs(x)).sum(1)
    u = 2.0 ** -24
    gamma = (in_dim + 3) * u / (1 - (in_dim + 3) * u)  # serial sum + up to three product roundings
    assert rc == 0 and np.all(np.abs(y - ex) <= gamma * absum)
    assert np.median(np.abs(y - ex)) < 0.05 * gamma * np.median(absum)
