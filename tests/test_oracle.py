"""Pins the CPU oracle (oracle/ssdq_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible restatement mistake (a swapped
nibble, a wrong shift in the Q4_K 6-bit unpacking, a dropped min term, a
round-half-even instead of half-away, a wrong GQA head map or block-table
index) fails it:
  * the reference's own known-answer tests for this path, restated;
  * exhaustive f16 widening against numpy's independent conversion;
  * encoder round trips (tests/encoders.py packs fields, the oracle decodes);
  * two-path agreement: dequantized elements reassembled into the serial
    fp32 sum reproduce the matvec bit for bit;
  * closed forms, float64 brute force and error bounds.
"""
import numpy as np
import pytest

import encoders as enc
import ssdq_oracle as o

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14


# --------------------------------------------------------------- type table
def test_type_table_matches_gguf():
    # src/model/gguf.rs:87-135
    assert (o.block_size(Q4_0), o.type_size(Q4_0)) == (32, 2 + 32 // 2)
    assert (o.block_size(Q8_0), o.type_size(Q8_0)) == (32, 2 + 32)
    assert (o.block_size(Q4_K), o.type_size(Q4_K)) == (256, 2 + 2 + 12 + 256 // 2)
    assert (o.block_size(Q6_K), o.type_size(Q6_K)) == (256, 256 // 2 + 256 // 4 + 256 // 16 + 2)
    assert o.block_size(3) == 0  # Q4_1 not on this path


# -------------------------------------------------------------- f16 -> f32
def test_f16_widening_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = o.f16_to_f32(h).view(np.uint32)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32)
    nan = np.isnan(h.view(np.float16))
    assert np.array_equal(ours[~nan], ref[~nan])
    # NaNs: same sign and payload, and quieted (half::f16::to_f32 sets the quiet bit)
    assert np.array_equal(ours[nan] | 0x00400000, ref[nan] | 0x00400000)
    assert np.all(ours[nan] & 0x00400000)


def test_f16_known_answer():
    # compute.rs:2557-2562: f16(3.14) round trip within 0.01
    bits = enc.f16_bits(3.14)
    assert abs(float(o.f16_to_f32(np.array([bits]))[0]) - 3.14) < 0.01
    # subnormal, max, -0
    assert o.f16_to_f32(np.array([0x0001], np.uint16))[0] == np.float32(2.0 ** -24)
    assert o.f16_to_f32(np.array([0x7BFF], np.uint16))[0] == np.float32(65504.0)
    assert o.f16_to_f32(np.array([0x8000], np.uint16)).view(np.uint32)[0] == 0x80000000


# ------------------------------------------------------- reference KATs
def test_matvec_q4_0_all_0x88_is_zero():
    # compute.rs:2347-2366
    blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), np.full(16, 0x88, np.uint8)])
    y, rc = o.matvec(Q4_0, blk, np.ones(32, np.float32), 1, 32)
    assert rc == 0 and abs(y[0]) < 1e-5


def test_matvec_q8_0_ones_is_32():
    # compute.rs:2369-2381
    blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), np.ones(32, np.uint8)])
    y, rc = o.matvec(Q8_0, blk, np.ones(32, np.float32), 1, 32)
    assert rc == 0 and abs(y[0] - 32.0) < 1e-3


def test_unsupported_dtype_zeros():
    # compute.rs:672-675 / streamer.rs:119-123
    y, rc = o.matvec(3, np.zeros(64, np.uint8), np.ones(32, np.float32), 2, 32)
    assert rc == 1 and np.all(y == 0)
    out, rc = o.dequantize(3, np.zeros(64, np.uint8), 32)
    assert rc == 1 and np.all(out == 0)


# ------------------------------------------------- encoder round trips
def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_q4_0_layout_round_trip():
    g = np.random.default_rng(1)
    blocks, want = [], []
    for i in range(64):
        d = enc.f16_bits(g.uniform(0.002, 0.02))
        q = np.roll(np.arange(-8, 8).repeat(2), i)  # every code at every position
        blocks.append(enc.enc_q4_0(d, q))
        want.append(enc.dec_expect_q4_0(d, q))
    got, rc = o.dequantize(Q4_0, np.concatenate(blocks), 64 * 32)
    assert rc == 0 and np.array_equal(_bits(got), _bits(np.concatenate(want)))


def test_q8_0_layout_round_trip():
    g = np.random.default_rng(2)
    blocks, want = [], []
    for i in range(16):
        d = enc.f16_bits(g.uniform(0.002, 0.02))
        q = np.arange(-128, 128)[i * 16:(i + 1) * 16].repeat(2)
        blocks.append(enc.enc_q8_0(d, q))
        want.append((q.astype(np.float32) * enc.f16_val(d)).astype(np.float32))
    got, rc = o.dequantize(Q8_0, np.concatenate(blocks), 16 * 32)
    assert rc == 0 and np.array_equal(_bits(got), _bits(np.concatenate(want)))


def test_q4_k_layout_round_trip_all_scale_values():
    # every 6-bit scale and min value at every sub-block position, both branches
    g = np.random.default_rng(3)
    blocks, want = [], []
    for i in range(64):
        d, dmin = enc.f16_bits(g.uniform(0.001, 0.01)), enc.f16_bits(g.uniform(0.001, 0.01))
        s = (i + 7 * np.arange(8)) % 64
        m = (3 * i + 11 * np.arange(8) + 5) % 64
        q = g.integers(0, 16, 256)
        blocks.append(enc.enc_q4_k(d, dmin, s, m, q))
        want.append(enc.dec_expect_q4_k(d, dmin, s, m, q))
    got, rc = o.dequantize(Q4_K, np.concatenate(blocks), 64 * 256)
    assert rc == 0 and np.array_equal(_bits(got), _bits(np.concatenate(want)))


def test_q4_k_high_bits_land_low():
    # sb >= 4 takes sc[sb-4] >> 6 as its LOW two bits (compute.rs:728-731):
    # s[4] = 1 (only the low bit) must decode as 1, not 16
    s = np.array([0, 0, 0, 0, 1, 0, 0, 0])
    blk = enc.enc_q4_k(enc.f16_bits(1.0), 0, s, np.zeros(8, int), np.ones(256, int))
    assert blk[4] == 0x40 and blk[12] == 0  # the bit sits in sc[0] bit 6
    got, _ = o.dequantize(Q4_K, blk, 256)
    assert np.all(got[128:160] == 1.0) and np.all(got[:128] == 0) and np.all(got[160:] == 0)


def test_q6_k_layout_round_trip():
    g = np.random.default_rng(4)
    blocks, want = [], []
    for i in range(16):
        d = enc.f16_bits(g.uniform(0.001, 0.01))
        sc = np.arange(-128, 128)[i * 16:(i + 1) * 16]
        q = np.roll(np.arange(-32, 32).repeat(4), 5 * i)
        blocks.append(enc.enc_q6_k(d, sc, q))
        want.append(enc.dec_expect_q6_k(d, sc, q))
    got, rc = o.dequantize(Q6_K, np.concatenate(blocks), 16 * 256)
    assert rc == 0 and np.array_equal(_bits(got), _bits(np.concatenate(want)))


def test_dequant_truncated_data_zero_fills():
    # streamer.rs: `break` when a block does not fit, then resize with zeros
    blk = enc.enc_q8_0(enc.f16_bits(1.0), np.arange(32) - 16)
    got, _ = o.dequantize(Q8_0, np.concatenate([blk, blk[:10]]), 96)
    assert np.array_equal(got[:32], np.arange(32, dtype=np.float32) - 16)
    assert np.all(got[32:] == 0)


# ------------------------------------------------ two-path agreement
def _serial_sum(terms):
    """fl(...fl(fl(0 + t0) + t1)...) per row, terms [rows, n] float32."""
    s = np.zeros(terms.shape[0], np.float32)
    for i in range(terms.shape[1]):
        s = (s + terms[:, i]).astype(np.float32)
    return s


@pytest.mark.parametrize("dtype,in_dim", [(Q4_0, 256), (Q8_0, 256), (Q6_K, 512), (Q4_K, 512)])
def test_matvec_equals_serial_sum_of_dequantized_elements(dtype, in_dim):
    from ssdq import synth
    out_dim = 24
    w = synth.quant_weights(dtype, out_dim, in_dim, 77)
    x = synth.normal_f32(in_dim, 78)
    y, rc = o.matvec(dtype, w, x, out_dim, in_dim)
    e, _ = o.dequantize(dtype, w, out_dim * in_dim)
    e = e.reshape(out_dim, in_dim)
    prod = (e * x[None, :]).astype(np.float32)
    if dtype == Q4_K:  # sum += v0*x[i] + v1*x[i+1]  (compute.rs:745)
        terms = (prod[:, 0::2] + prod[:, 1::2]).astype(np.float32)
    else:              # sum += elem * x[i]
        terms = prod
    assert rc == 0 and np.array_equal(_bits(y), _bits(_serial_sum(terms)))


def test_matvec_mt_bit_identical():
    from ssdq import synth
    w = synth.quant_weights(Q4_K, 64, 1024, 5)
    x = synth.normal_f32(1024, 6)
    a, _ = o.matvec(Q4_K, w, x, 64, 1024)
    b, _ = o.matvec(Q4_K, w, x, 64, 1024, threads=5)
    assert np.array_equal(_bits(a), _bits(b))


def test_q4_k_closed_form():
    # d = 1, dmin = 0.5, s = 1..8, m = 0..7, q = j % 16, x = 1:
    # y = sum_sb (s_sb * sum_j q_j - 0.5 * m_sb * 32), exact in fp32
    s, m = np.arange(1, 9), np.arange(8)
    q = np.arange(256) % 16
    blk = enc.enc_q4_k(enc.f16_bits(1.0), enc.f16_bits(0.5), s, m, q)
    y, _ = o.matvec(Q4_K, blk, np.ones(256, np.float32), 1, 256)
    qsum = q.reshape(8, 32).sum(1)
    assert y[0] == float((s * qsum).sum() - 0.5 * (m * 32).sum())


@pytest.mark.parametrize("dtype,in_dim", [(Q4_0, 4096), (Q8_0, 4096), (Q4_K, 4096), (Q6_K, 4096)])
def test_matvec_within_fp32_bound_of_exact(dtype, in_dim):
    from ssdq import synth
    out_dim = 64
    w = synth.quant_weights(dtype, out_dim, in_dim, 11)
    x = synth.normal_f32(in_dim, 12)
    y, _ = o.matvec(dtype, w, x, out_dim, in_dim)
    ex = o.matvec_exact(dtype, w, x, out_dim, in_dim)
    e, _ = o.dequantize(dtype, w, out_dim * in_dim)
    absum = (np.abs(e.reshape(out_dim, in_dim).astype(np.float64)) * np.abs(x)).sum(1)
    u = 2.0 ** -24
    gamma = (in_dim + 2) * u / (1 - (in_dim + 2) * u)  # serial-sum + product rounding bound
    assert np.all(np.abs(y - ex) <= gamma * absum)
    # and the bound is not vacuous: typical error is far below it
    assert np.median(np.abs(y - ex)) < 0.05 * gamma * np.median(absum)


# -------------------------------------------------------- INT8 quantizer
def _quantize_np(rows):
    """Independent restatement in float64 arithmetic on float32 values."""
    rows = np.asarray(rows, np.float32)
    a = np.abs(rows)
    a = np.where(np.isnan(a), 0, a)
    absmax = a.max(axis=1).astype(np.float32)
    codes = np.zeros(rows.shape, np.int8)
    scales = np.zeros(rows.shape[0], np.float32)
    for r in range(rows.shape[0]):
        am = absmax[r]
        if am == 0:
            continue
        with np.errstate(all="ignore"):
            inv = np.float32(127.0) / am
            scales[r] = am / np.float32(127.0)
            t = (rows[r] * inv).astype(np.float32).astype(np.float64)
            rnd = np.sign(t) * np.floor(np.abs(t) + 0.5)  # half away from zero (exact in f64)
        rnd = np.where(np.isnan(rnd), 0, np.clip(rnd, -127, 127))
        codes[r] = rnd.astype(np.int8)
    return codes, scales


def test_int8_quantizer_matches_independent_restatement():
    g = np.random.default_rng(9)
    rows = g.standard_normal((512, 1024)).astype(np.float32)
    rows[3] *= 1e-30  # tiny rows (inv overflows towards inf scale)
    rows[4] = 0
    rows[5, :7] = np.nan
    rows[6, 10] = np.inf
    rows[7] = -rows[8]
    rows[9, 100] = -1e38
    c, s = o.quantize_rows(rows, 512, 1024)
    c2, s2 = _quantize_np(rows)
    assert np.array_equal(c, c2.ravel())
    assert np.array_equal(s.view(np.uint32), s2.view(np.uint32))


def test_int8_ties_round_away_from_zero():
    # absmax 127 -> inv = 1 exactly; v = k + 0.5 ties
    row = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5], np.float32)
    c, s = o.quantize_rows(row, 1, row.size)
    assert list(c) == [127, 1, -1, 2, -2, 3, -3, 127] and s[0] == np.float32(1.0)


def test_int8_extremes_and_symmetry():
    g = np.random.default_rng(10)
    row = g.standard_normal(256).astype(np.float32)
    c, s = o.quantize_rows(row, 1, 256)
    i = int(np.argmax(np.abs(row)))
    assert abs(int(c[i])) == 127 and np.sign(c[i]) == np.sign(row[i])
    cn, sn = o.quantize_rows(-row, 1, 256)
    assert np.array_equal(cn, -c) and sn[0] == s[0]
    # scale * 127 recovers absmax to within one rounding
    assert abs(float(s[0]) * 127 - float(np.abs(row).max())) <= 2 * np.spacing(np.float32(np.abs(row).max()))


def test_int8_reference_known_answers():
    # quantized_kv_cache.rs:243-260: (i - 64) * 0.1, error < scale + 0.01
    v = ((np.arange(128) - 64) * 0.1).astype(np.float32)
    c, s = o.quantize_rows(v, 1, 128)
    d = o.dequantize_rows(c, s, 1, 128)
    assert np.all(np.abs(v - d) < s[0] + 0.01)
    # quantized_kv_cache.rs:263-269 / block_swap.rs:1014-1025: zeros -> scale 0, codes 0
    c, s = o.quantize_rows(np.zeros(16, np.float32), 2, 8)
    assert np.all(s == 0) and np.all(c == 0) and np.all(o.dequantize_rows(c, s, 2, 8) == 0)
    # quantized_kv_cache.rs:344-359: dequantize_into(64, 64) == dequantize()[64..128]
    v = ((np.arange(256) - 128) * 0.05).astype(np.float32)
    c, s = o.quantize_rows(v, 1, 256)
    full = o.dequantize_rows(c, s, 1, 256)
    sl = (c[64:128].astype(np.float32) * s[0]).astype(np.float32)
    assert np.all(np.abs(sl - full[64:128]) < 1e-6)
    # block_swap.rs:996-1011: (i - 128) * 0.01, dim 64, error < 0.02
    v = ((np.arange(256) - 128) * 0.01).astype(np.float32)
    c, s = o.quantize_rows(v, 4, 64)
    assert np.all(np.abs(o.dequantize_rows(c, s, 4, 64) - v) < 0.02)
    # quantized_kv_cache.rs:272-289: key of ones dequantizes within 0.05 of 1.0
    c, s = o.quantize_rows(np.ones(256, np.float32), 1, 256)
    assert abs(float(o.dequantize_rows(c, s, 1, 256)[0]) - 1.0) < 0.05
    # block_swap.rs:1100-1135: 1.5 and -0.75 rows recover within 0.02
    for val in (1.5, -0.75):
        c, s = o.quantize_rows(np.full(32, val, np.float32), 4, 8)
        assert np.all(np.abs(o.dequantize_rows(c, s, 4, 8) - val) < 0.02)


# -------------------------------------------------------------- attention
def _attn_double(q, K, V):
    """Two-pass softmax attention in float64 for one head."""
    s = (K.astype(np.float64) @ q.astype(np.float64)) / np.sqrt(q.size)
    w = np.exp(s - s.max())
    return (w[:, None] * V.astype(np.float64)).sum(0) / w.sum()


def _paged_case(g, n_seq, n_head, n_kv, hd, bs, ctx_lens, max_blocks):
    n_phys = n_seq * max_blocks
    kv_dim = n_kv * hd
    kc = g.integers(-127, 128, (n_phys * bs, kv_dim)).astype(np.int8)
    vc = g.integers(-127, 128, (n_phys * bs, kv_dim)).astype(np.int8)
    ks = g.uniform(0.005, 0.03, n_phys * bs).astype(np.float32)
    vs = g.uniform(0.005, 0.03, n_phys * bs).astype(np.float32)
    tables = g.permutation(n_phys).astype(np.int32).reshape(n_seq, max_blocks)
    q = g.standard_normal((n_seq, n_head, hd)).astype(np.float32)
    return q, kc, ks, vc, vs, tables, np.asarray(ctx_lens, np.int32)


def test_paged_attention_matches_double_two_pass():
    g = np.random.default_rng(21)
    n_seq, n_head, n_kv, hd, bs, mb = 3, 8, 2, 64, 16, 8
    ctx = [1, 37, 128]
    q, kc, ks, vc, vs, tables, cl = _paged_case(g, n_seq, n_head, n_kv, hd, bs, ctx, mb)
    out = o.paged_attention_int8(q, kc, ks, vc, vs, tables, cl, n_seq, n_head, n_kv, hd, bs, mb)
    out = out.reshape(n_seq, n_head, hd)
    group = n_head // n_kv
    for s in range(n_seq):
        p = np.arange(ctx[s])
        rows = tables[s, p // bs] * bs + p % bs
        for h in range(n_head):
            kh = h // group
            K = kc[rows, kh * hd:(kh + 1) * hd].astype(np.float32) * ks[rows, None]
            V = vc[rows, kh * hd:(kh + 1) * hd].astype(np.float32) * vs[rows, None]
            ref = _attn_double(q[s, h], K.astype(np.float32), V.astype(np.float32))
            np.testing.assert_allclose(out[s, h], ref, rtol=1e-5, atol=1e-6)


def test_paged_attention_single_token_is_v():
    # flash_attention.rs:407-459: one position -> softmax weight 1 -> out == V
    g = np.random.default_rng(22)
    q, kc, ks, vc, vs, tables, cl = _paged_case(g, 2, 4, 4, 128, 16, [1, 1], 2)
    out = o.paged_attention_int8(q, kc, ks, vc, vs, tables, cl, 2, 4, 4, 128, 16, 2).reshape(2, 4, 128)
    for s in range(2):
        row = tables[s, 0] * 16
        v = (vc[row].astype(np.float32) * vs[row]).astype(np.float32).reshape(4, 128)
        assert np.array_equal(out[s], v)


def test_paged_block_table_mapping():
    # paged_attention.rs:1187-1198: table [5, 12, 3], block 4:
    # positions 0..9 live in physical rows 20-23, 48-51, 12-13.
    # V row = its physical row id, q = 0 -> uniform weights -> out = mean row id
    n_phys, bs, hd = 16, 4, 64
    kc = np.zeros((n_phys * bs, hd), np.int8)
    vc = np.repeat(np.arange(n_phys * bs, dtype=np.int8)[:, None], hd, 1)
    ones = np.ones(n_phys * bs, np.float32)
    tables = np.array([[5, 12, 3]], np.int32)
    out = o.paged_attention_int8(np.zeros(hd, np.float32), kc, ones, vc, ones, tables,
                                 np.array([10], np.int32), 1, 1, 1, hd, bs, 3)
    rows = [20, 21, 22, 23, 48, 49, 50, 51, 12, 13]
    np.testing.assert_allclose(out, np.mean(rows), rtol=1e-6)


def test_gqa_head_map():
    # kv_h = h / (n_head / n_head_kv) (flash_attention.rs:71-77): V of kv head j == j
    n_head, n_kv, hd, seq = 8, 2, 64, 5
    k = np.zeros((seq, n_kv, hd), np.float32)
    v = np.zeros((seq, n_kv, hd), np.float32)
    v[:, 1, :] = 1.0
    out = o.flash_attention_f32(np.zeros((n_head, hd), np.float32), k, v, n_head, n_kv, hd, seq, 0, seq)
    out = out.reshape(n_head, hd)
    assert np.all(out[:4] == 0) and np.all(out[4:] == 1)


def test_flash_attention_window_and_empty():
    g = np.random.default_rng(23)
    n_head, n_kv, hd, seq = 4, 2, 64, 40
    q = g.standard_normal((n_head, hd)).astype(np.float32)
    k = g.standard_normal((seq, n_kv, hd)).astype(np.float32)
    v = g.standard_normal((seq, n_kv, hd)).astype(np.float32)
    out = o.flash_attention_f32(q, k, v, n_head, n_kv, hd, seq, 7, 99).reshape(n_head, hd)
    for h in range(n_head):
        ref = _attn_double(q[h], k[7:, h // 2], v[7:, h // 2])
        np.testing.assert_allclose(out[h], ref, rtol=1e-5, atol=1e-6)
    empty = o.flash_attention_f32(q, k, v, n_head, n_kv, hd, seq, 30, 30)
    assert np.all(empty == 0)


def test_paged_attention_window_matches_double_two_pass():
    # flash_attention_windowed (flash_attention.rs:146-227): positions
    # window_start .. min(window_end, seq_len) per sequence, zeros when empty;
    # pinned against two-pass double-precision attention over exactly those
    # rows, and a full window against the unwindowed oracle bit for bit
    g = np.random.default_rng(24)
    n_seq, n_head, n_kv, hd, bs, mb = 5, 8, 2, 64, 16, 8
    ctx = [100, 37, 128, 60, 90]
    lo = np.array([13, 0, 127, 70, 5], np.int32)   # seq 3: start past ctx -> empty
    hi = np.array([99, 20, 500, 80, 5], np.int32)  # seq 2: end past ctx; seq 4: empty
    q, kc, ks, vc, vs, tables, cl = _paged_case(g, n_seq, n_head, n_kv, hd, bs, ctx, mb)
    out = o.paged_attention_int8_window(q, kc, ks, vc, vs, tables, cl, lo, hi, n_seq, n_head, n_kv, hd, bs, mb)
    out = out.reshape(n_seq, n_head, hd)
    group = n_head // n_kv
    for s in range(n_seq):
        p = np.arange(lo[s], min(hi[s], ctx[s]))
        if p.size == 0:
            assert np.all(out[s] == 0), s
            continue
        rows = tables[s, p // bs] * bs + p % bs
        for h in range(n_head):
            kh = h // group
            K = kc[rows, kh * hd:(kh + 1) * hd].astype(np.float32) * ks[rows, None]
            V = vc[rows, kh * hd:(kh + 1) * hd].astype(np.float32) * vs[rows, None]
            ref = _attn_double(q[s, h], K.astype(np.float32), V.astype(np.float32))
            np.testing.assert_allclose(out[s, h], ref, rtol=1e-5, atol=1e-6)
    full = o.paged_attention_int8_window(q, kc, ks, vc, vs, tables, cl, np.zeros(n_seq, np.int32),
                                         cl.copy(), n_seq, n_head, n_kv, hd, bs, mb)
    plain = o.paged_attention_int8(q, kc, ks, vc, vs, tables, cl, n_seq, n_head, n_kv, hd, bs, mb)
    assert np.array_equal(full.view(np.uint32), plain.view(np.uint32))
    nowin = o.paged_attention_int8_window(q, kc, ks, vc, vs, tables, cl, None, None, n_seq, n_head, n_kv, hd, bs,
                                          mb)
    assert np.array_equal(nowin.view(np.uint32), plain.view(np.uint32))


def test_online_softmax_large_scores_finite():
    # flash_attention.rs:461-488: large inputs stay finite
    hd = 64
    q = np.full((1, hd), 100.0, np.float32)
    k = np.full((3, 1, hd), 100.0, np.float32)
    v = np.ones((3, 1, hd), np.float32)
    out = o.flash_attention_f32(q, k, v, 1, 1, hd, 3, 0, 3)
    assert np.all(np.isfinite(out)) and np.allclose(out, 1.0)


# ------------------------------------------------------------------- GEMM
def test_gemm_oracle_is_per_token_matvec_of_widened_bf16():
    from ssdq import synth
    M, N, K = 6, 32, 512
    w = synth.quant_weights(Q4_K, N, K, 31)
    xf = synth.normal_f32((M, K), 32)
    xb = synth.f32_to_bf16_bits(xf)
    y = o.gemm_q4k_bf16(w, xb, M, N, K, threads=3).reshape(M, N)
    widened = (xb.astype(np.uint32) << 16).view(np.float32)
    for t in range(M):
        yt, _ = o.matvec(Q4_K, w, widened[t], N, K)
        assert np.array_equal(y[t].view(np.uint32), yt.view(np.uint32))


def test_bf16_rounding_helper():
    from ssdq import synth
    # ties to even: 1 + 2^-8 -> 1.0, 1 + 3*2^-8 -> 1 + 2^-6; exact values kept
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5], np.float32)
    r = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(x))
    assert list(r) == [1.0, 1.0, 1.015625, -2.5]


# ------------------------------------------------- INT8 KV swap slots
def test_kv_swap_slot_reference_known_answers():
    # block_swap.rs:1177-1185: 16 x 128 -> 4228 bytes, f32 16388 (ratio ~3.88)
    assert o.kv_slot_bytes(16, 128) == 4228
    assert 3.0 < (16 * 128 * 2 * 4 + 4) / o.kv_slot_bytes(16, 128) < 4.5
    # block_swap.rs:1028-1066: write / read within INT8 error, num_filled kept
    bs, kv = 4, 8
    keys = ((np.arange(bs * kv) - 16.0) * 0.1).astype(np.float32)
    vals = ((np.arange(bs * kv) - 16.0) * 0.05).astype(np.float32)
    k, v, nf = o.kv_swap_read(o.kv_swap_write(keys, vals, bs, kv, 3), bs, kv)
    assert nf == 3 and np.all(np.abs(k - keys) < 0.02) and np.all(np.abs(v - vals) < 0.02)


def test_kv_swap_slot_layout():
    # codes K | codes V | scales K | scales V | num_filled (block_swap.rs:14-15, 228-252),
    # checked against the quantizer's own outputs placed by numpy
    g = np.random.default_rng(8)
    bs, kv = 16, 1024
    keys = g.standard_normal(bs * kv).astype(np.float32)
    vals = g.standard_normal(bs * kv).astype(np.float32)
    slot = o.kv_swap_write(keys, vals, bs, kv, 0xA1B2C3D4)
    kc, ks = o.quantize_rows(keys, bs, kv)
    vc, vs = o.quantize_rows(vals, bs, kv)
    want = np.concatenate([kc.view(np.uint8).ravel(), vc.view(np.uint8).ravel(), ks.view(np.uint8),
                           vs.view(np.uint8), np.array([0xD4, 0xC3, 0xB2, 0xA1], np.uint8)])
    assert np.array_equal(slot, want)
    k, v, nf = o.kv_swap_read(slot, bs, kv)
    assert nf == 0xA1B2C3D4
    assert np.array_equal(k, o.dequantize_rows(kc, ks, bs, kv).ravel())
