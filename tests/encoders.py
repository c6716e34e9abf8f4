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
  Q2_K  d f16 @0, dmin f16 @2, sc[16] @4 (low nibble scale, high nibble min of
        16-element sub-block i), qs[64] @20: element i = bits 2*(i%4) of qs[i/4]
                                                      (compute.rs:927-966)
  Q3_K  hmask[32] @0, qs[64] @32, sc[12] @96, d f16 @108: element i = (bits
        2*(i%4) of qs[i/4] | bit i%8 of hmask[i/8] << 2) - 4; 6-bit signed scale
        of sub-block sb: low four bits = nibble sb&1 of sc[sb/2], high two bits
        = bits 2*(sb%4) of sc[8+sb/4]                 (compute.rs:793-840)
  Q5_K  d @0, dmin @2, sc[12] @4 (Q4_K packing), qh[32] @16, ql[128] @48:
        element sb*32+2j = low nibble of ql[sb*16+j], +1 = high nibble, each
        with bit (i%8) of qh[i/8] as bit 4             (compute.rs:842-902)
  Q8_K  d f32 @0, int8 qs[256] @4, 16 int16 bsums @260 (not read)
                                                      (compute.rs:968-993)
  IQ4_NL d f16 @0, qs[16] @2: element 2j / 2j+1 = code book entry of the low /
        high nibble of qs[j]                          (compute.rs:995-1028)
  IQ4_XS d f16 @0, scales_h u16 @2, scales_l u16[8] @4, qs[128] @20: 6-bit
        scale of sub-block sb = nibble sb%2 of scales_l[sb/2] | bits 2sb of
        scales_h << 4, minus 32; elements as IQ4_NL    (compute.rs:1030-1077)
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


# IQ4_NL code book: a format constant (compute.rs:997-999)
IQ4_NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                  np.int64)


def _put_f16(b, off, bits):
    b[off], b[off + 1] = int(bits) & 0xFF, int(bits) >> 8


def _pack2(q):
    """four 2-bit fields per byte, field i of byte j = element 4j+i"""
    q = np.asarray(q, np.int64)
    return (q[0::4] | (q[1::4] << 2) | (q[2::4] << 4) | (q[3::4] << 6)).astype(np.uint8)


def _pack_bits(bits):
    """one bit per element, bit i%8 of byte i/8"""
    bits = np.asarray(bits, np.int64).reshape(-1, 8)
    return (bits << np.arange(8)).sum(axis=1).astype(np.uint8)


def _q4k_scales(s, m):
    s = np.asarray(s, np.int64)
    m = np.asarray(m, np.int64)
    sc = np.zeros(12, np.int64)
    for i in range(4):
        sc[i] = s[i] | ((s[i + 4] & 3) << 6)
        sc[i + 4] = m[i] | ((m[i + 4] & 3) << 6)
        sc[i + 8] = (s[i + 4] >> 2) | ((m[i + 4] >> 2) << 4)
    return sc.astype(np.uint8)


def enc_q2_k(d_bits, dmin_bits, s, m, q):
    """s, m: 16 ints in [0, 15]; q: 256 ints in [0, 3]."""
    b = np.zeros(84, np.uint8)
    _put_f16(b, 0, d_bits)
    _put_f16(b, 2, dmin_bits)
    b[4:20] = (np.asarray(s, np.int64) | (np.asarray(m, np.int64) << 4)).astype(np.uint8)
    b[20:84] = _pack2(q)
    return b


def dec_expect_q2_k(d_bits, dmin_bits, s, m, q):
    d, dmin = f16_val(d_bits), f16_val(dmin_bits)
    S = np.repeat((d * np.asarray(s, np.float32)).astype(np.float32), 16)
    M = np.repeat((dmin * np.asarray(m, np.float32)).astype(np.float32), 16)
    return ((S * np.asarray(q, np.float32)).astype(np.float32) - M).astype(np.float32)


def enc_q3_k(d_bits, sv, q):
    """sv: 16 ints in [-32, 31]; q: 256 ints in [-4, 3]."""
    u = np.asarray(q, np.int64) + 4
    assert u.min() >= 0 and u.max() <= 7
    s6 = np.asarray(sv, np.int64) & 63
    b = np.zeros(110, np.uint8)
    b[0:32] = _pack_bits(u >> 2)
    b[32:96] = _pack2(u & 3)
    sc = np.zeros(12, np.int64)
    for sb in range(16):
        sc[sb // 2] |= (s6[sb] & 15) << (4 * (sb & 1))
        sc[8 + sb // 4] |= (s6[sb] >> 4) << (2 * (sb % 4))
    b[96:108] = sc.astype(np.uint8)
    _put_f16(b, 108, d_bits)
    return b


def dec_expect_q3_k(d_bits, sv, q):
    S = np.repeat((f16_val(d_bits) * np.asarray(sv, np.float32)).astype(np.float32), 16)
    return (S * np.asarray(q, np.float32)).astype(np.float32)


def enc_q5_k(d_bits, dmin_bits, s, m, q):
    """s, m: 8 six-bit ints; q: 256 ints in [0, 31]."""
    q = np.asarray(q, np.int64)
    b = np.zeros(176, np.uint8)
    _put_f16(b, 0, d_bits)
    _put_f16(b, 2, dmin_bits)
    b[4:16] = _q4k_scales(s, m)
    b[16:48] = _pack_bits(q >> 4)
    lo = q & 15
    b[48:176] = (lo[0::2] | (lo[1::2] << 4)).astype(np.uint8)
    return b


def dec_expect_q5_k(d_bits, dmin_bits, s, m, q):
    d, dmin = f16_val(d_bits), f16_val(dmin_bits)
    S = np.repeat((d * np.asarray(s, np.float32)).astype(np.float32), 32)
    M = np.repeat((dmin * np.asarray(m, np.float32)).astype(np.float32), 32)
    return ((S * np.asarray(q, np.float32)).astype(np.float32) - M).astype(np.float32)


def enc_q8_k(d, q):
    """d: f32 scale; q: 256 ints in [-128, 127]."""
    q = np.asarray(q, np.int64)
    b = np.zeros(292, np.uint8)
    b[0:4] = np.array([d], np.float32).view(np.uint8)
    b[4:260] = q.astype(np.int8).view(np.uint8)
    b[260:292] = q.reshape(16, 16).sum(axis=1).astype(np.int16).view(np.uint8)
    return b


def dec_expect_q8_k(d, q):
    return (np.float32(d) * np.asarray(q, np.float32)).astype(np.float32)


def enc_iq4_nl(d_bits, idx):
    """idx: 32 code-book indices in [0, 15]."""
    idx = np.asarray(idx, np.int64)
    b = np.zeros(18, np.uint8)
    _put_f16(b, 0, d_bits)
    b[2:18] = (idx[0::2] | (idx[1::2] << 4)).astype(np.uint8)
    return b


def dec_expect_iq4_nl(d_bits, idx):
    return (f16_val(d_bits) * IQ4_NL[np.asarray(idx)].astype(np.float32)).astype(np.float32)


def enc_iq4_xs(d_bits, s6, idx):
    """s6: 8 six-bit scale codes (scale = s6 - 32); idx: 256 indices in [0, 15]."""
    s6 = np.asarray(s6, np.int64)
    idx = np.asarray(idx, np.int64)
    b = np.zeros(148, np.uint8)
    _put_f16(b, 0, d_bits)
    sh = int(sum(int(s6[sb] >> 4) << (2 * sb) for sb in range(8)))
    b[2], b[3] = sh & 0xFF, sh >> 8
    for sb in range(8):
        b[4 + (sb // 2) * 2] |= (s6[sb] & 15) << (4 * (sb % 2))
    b[20:148] = (idx[0::2] | (idx[1::2] << 4)).astype(np.uint8)
    return b


def dec_expect_iq4_xs(d_bits, s6, idx):
    ds = (f16_val(d_bits) * (np.asarray(s6, np.float32) - np.float32(32))).astype(np.float32)
    return (np.repeat(ds, 32) * IQ4_NL[np.asarray(idx)].astype(np.float32)).astype(np.float32)
