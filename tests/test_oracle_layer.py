"""Pins the oracle's decode-layer f32 ops (RoPE, SiLU, RMSNorm and the fused
variants; src/metal/compute.rs:482-645) with the reference's own tests and with
what the mathematics fixes: RoPE at position 0 is the identity, acts on
adjacent pairs, rotates pair i by position * theta^(-2i/head_dim) (checked in
double precision), preserves pair norms and composes additively; SiLU is
x * sigmoid(x); RMSNorm output has unit RMS and is scale invariant."""
import math

import numpy as np

import encoders as enc
import ssdq_oracle as o

Q8_0 = 8


def test_rope_reference_known_answers():
    # compute.rs:3301-3313: position 0 is the identity
    x = np.arange(1, 9, dtype=np.float32)
    assert np.array_equal(o.rope_multi_head(x, 4, 2, 0, 10000.0), x)
    # compute.rs:3265-3298, values from the formula in double precision
    head_dim, n_heads, pos, theta = 4, 3, 7, 10000.0
    x = (np.arange(n_heads * head_dim, dtype=np.float32) + 1) * 0.5
    got = o.rope_multi_head(x, head_dim, n_heads, pos, theta)
    for h in range(n_heads):
        for i in range(head_dim // 2):
            a = pos / theta ** (2 * i / head_dim)
            x0, x1 = float(x[h * 4 + 2 * i]), float(x[h * 4 + 2 * i + 1])
            assert abs(got[h * 4 + 2 * i] - (x0 * math.cos(a) - x1 * math.sin(a))) < 1e-5
            assert abs(got[h * 4 + 2 * i + 1] - (x0 * math.sin(a) + x1 * math.cos(a))) < 1e-5


def test_rope_pairs_are_adjacent_and_rotations_compose():
    g = np.random.default_rng(1)
    hd = 128
    # a unit vector at index 2i only moves indices 2i, 2i+1
    for i in (0, 5, 63):
        e = np.zeros(hd, np.float32)
        e[2 * i] = 1.0
        r = o.rope_multi_head(e, hd, 1, 1234, 500000.0)
        moved = np.flatnonzero(r != e)
        assert set(moved) <= {2 * i, 2 * i + 1}
    # pair norms are kept, and rotating by p1 then p2 equals rotating by p1 + p2
    x = g.standard_normal(4 * hd).astype(np.float32)
    r = o.rope_multi_head(x, hd, 4, 321, 10000.0)
    assert np.allclose(np.hypot(r[0::2], r[1::2]), np.hypot(x[0::2], x[1::2]), rtol=1e-5)
    two = o.rope_multi_head(o.rope_multi_head(x, hd, 4, 5, 10000.0), hd, 4, 9, 10000.0)
    assert np.allclose(two, o.rope_multi_head(x, hd, 4, 14, 10000.0), atol=2e-5)


def test_silu_reference_and_closed_form():
    s = o.silu(np.array([0.0, 1.0, -1.0], np.float32))
    assert abs(s[0]) < 1e-6 and s[1] > 0.5 and -0.5 < s[2] < 0.0  # compute.rs:2337-2344
    x = np.linspace(-30, 30, 1001).astype(np.float32)
    want = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.allclose(o.silu(x), want, rtol=1e-6, atol=1e-30)


def test_rmsnorm_reference_and_invariants():
    x = o.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 1e-5)
    assert abs(x[0] - 1 / math.sqrt(30 / 4 + 1e-5)) < 1e-4  # compute.rs:2327-2335
    g = np.random.default_rng(2)
    v = g.standard_normal(4096).astype(np.float32)
    r = o.rmsnorm(v, np.ones(4096, np.float32), 1e-6)
    assert abs(math.sqrt(np.mean(r.astype(np.float64) ** 2)) - 1) < 1e-5
    assert np.allclose(o.rmsnorm(v * 8, np.ones(4096, np.float32), 0.0), o.rmsnorm(v, np.ones(4096, np.float32), 0.0),
                       rtol=1e-5, atol=1e-6)


def test_post_attn_norm_reference_known_answers():
    # compute.rs:3458-3491
    n = 64
    hidden = np.arange(n, dtype=np.float32) * np.float32(0.1)
    attn = (n - np.arange(n)).astype(np.float32) * np.float32(0.05)
    w = (0.8 + (np.arange(n) % 3) * 0.1).astype(np.float32)
    h, out = o.fused_post_attn_norm(hidden, attn, w, 1e-5)
    assert np.allclose(h, np.arange(n) * 0.1 + (n - np.arange(n)) * 0.05, atol=1e-5)
    inv = 1 / math.sqrt(float((h.astype(np.float64) ** 2).sum()) / n + 1e-5)
    assert np.allclose(out, h * inv * w, atol=1e-5)


def test_fused_rmsnorm_linear_is_norm_then_projection():
    # compute.rs:3399-3427 with the projection as Q8_0 rows selecting one element:
    # logits[r] = x[r] * inv_rms * w[r], in double precision
    n, vocab = 64, 8
    g = np.random.default_rng(3)
    x = g.standard_normal(n).astype(np.float32)
    w = (0.5 + (np.arange(n) % 5) * 0.2).astype(np.float32)
    rows = []
    for r in range(vocab):
        q = np.zeros(n, np.int64)
        q[r] = 1
        rows.append(np.concatenate([enc.enc_q8_0(enc.f16_bits(1.0), q[b * 32:(b + 1) * 32]) for b in range(n // 32)]))
    y, rc = o.fused_rmsnorm_linear(Q8_0, np.concatenate(rows), x, w, vocab, n)
    inv = 1 / math.sqrt(float((x.astype(np.float64) ** 2).sum()) / n + 1e-5)
    assert rc == 0 and np.allclose(y, x[:vocab] * inv * w[:vocab], rtol=1e-6)
