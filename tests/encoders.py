"""Independent encoders for the reference's GGUF block layouts.

Each encoder packs chosen integer fields into block bytes, written as the
inverse of the reference's decoder.  Decoding what they produce must give back
the fields, so a wrong shift, nibble order or byte offset in the oracle (or
the device kernels) fails a round trip.

Layouts (reference):
  Q4_0  d f16 @0, qs[16] @2; element 2j = low nibble of qs[j] - 8, 2j+1 = high
        nibble - 8                                   (compute.rs:689-699)
  Q8_0  d f16 @0, int8 qs[32] @2                      (compute.rs:911-920)
  Q4_K  d f16 @0, dmin f16 @2, sc[12] @4, qs[128] @16. sub-block sb < 4:
        s = sc[sb] & 63, m = sc[sb+4] & 63; sb >= 4: s = (sc[sb-4] >> 6) |
        ((sc[sb+4] & 15) << 2), m = (sc[sb] >> 6) | ((sc[sb+4] >> 4) << 2);
        element sb*32+2j = low nibble of qs[sb*16+j], +1 = high nibble
                                                      (compute.rs:716-744)
  Q6_K  ql[128] @0, qh[64] @128, int8 scales[16] @192, d f16 @208; element i:
        q = (lo4 | hi2 << 4) - 32 with lo4 the (i&1 ? high : low) nibble of
        ql[i/2] and hi2 bits 2*(i%4) of qh[i/4], scale scales[i/16]
                                                      (compute.rs:764-785)
"""
import numpy as np


def f16_bits(v):
    return np.float16(v).view(np.uint16)


def f16_val(bits):
    return np.uint16(bits).view(np.float16).astype(np.float32)


def enc_q4_0(d_bits, q):
    """q: 32 ints in [-8, 7]."""
    q = np.asarray(q, np.int64) + 8
    assert q.min() >= 0 and q.max() <= 15
    b = np.zeros(18, np.uint8)
    b[0], b[1] = d_bits & 0xFF, d_bits >> 8
    b[2:18] = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    return b


def dec_expect_q4_0(d_bits, q):
    return np.float32(np.asarray(q, np.float32)) * f16_val(d_bits)


def enc_q8_0(d_bits, q):
    q = np.asarray(q, np.int64)
    b = np.zeros(34, np.uint8)
    b[0], b[1] = d_bits & 0xFF, d_bits >> 8
    b[2:34] = q.astype(np.int8).view(np.uint8)
    return b


def enc_q4_k(d_bits, dmin_bits, s, m, q):
    """s, m: 8 six-bit ints; q: 256 ints in [0, 15]."""
    s = np.asarray(s, np.int64)
    m = np.asarray(m, np.int64)
    q = np.asarray(q, np.int64)
    b = np.zeros(144, np.uint8)
    b[0], b[1] = d_bits & 0xFF, d_bits >> 8
    b[2], b[3] = dmin_bits & 0xFF, dmin_bits >> 8
    sc = np.zeros(12, np.int64)
    for i in range(4):
        # sub-blocks 0-3: low six bits of sc[i] / sc[i+4]
        # sub-blocks 4-7: their LOW two bits sit in bits 6-7 of sc[i] / sc[i+4],
        # the high four bits in the low / high nibble of sc[i+8]
        sc[i] = s[i] | ((s[i + 4] & 3) << 6)
        sc[i + 4] = m[i] | ((m[i + 4] & 3) << 6)
        sc[i + 8] = (s[i + 4] >> 2) | ((m[i + 4] >> 2) << 4)
    b[4:16] = sc.astype(np.uint8)
    b[16:144] = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    return b


def dec_expect_q4_k(d_bits, dmin_bits, s, m, q):
    d, dmin = f16_val(d_bits), f16_val(dmin_bits)
    S = (d * np.asarray(s, np.float32)).astype(np.float32)
    M = (dmin * np.asarray(m, np.float32)).astype(np.float32)
    S = np.repeat(S, 32)
    M = np.repeat(M, 32)
    return ((S * np.asarray(q, np.float32)).astype(np.float32) - M).astype(np.float32)


def enc_q6_k(d_bits, scales, q):
    """scales: 16 ints in [-128, 127]; q: 256 ints in [-32, 31]."""
    u = np.asarray(q, np.int64) + 32
    assert u.min() >= 0 and u.max() <= 63
    b = np.zeros(210, np.uint8)
    lo, hi = u & 15, u >> 4
    b[0:128] = (lo[0::2] | (lo[1::2] << 4)).astype(np.uint8)
    b[128:192] = (hi[0::4] | (hi[1::4] << 2) | (hi[2::4] << 4) | (hi[3::4] << 6)).astype(np.uint8)
    b[192:208] = np.asarray(scales, np.int64).astype(np.int8).view(np.uint8)
    b[208], b[209] = d_bits & 0xFF, d_bits >> 8
    return b


def dec_expect_q6_k(d_bits, scales, q):
    d = f16_val(d_bits)
    ds = (d * np.asarray(scales, np.float32)).astype(np.float32)
    return (np.repeat(ds, 16) * np.asarray(q, np.float32)).astype(np.float32)
