"""Fused dequant-matvec parity (matvec_*_cpu, src/metal/compute.rs:680-925).

Tolerance: |gpu - ref| <= 1e-4 + 1e-3 |ref| against the serial fp32 oracle,
with the exact-sum substitution of helpers.assert_close_attributed where the
reference's own fp32 chain is off by more than half a tolerance.
"""
import numpy as np
import pytest
import torch

import encoders as enc
import ssdq
import ssdq_oracle as o
from helpers import (announce, assert_close, assert_close_attributed, empty_dev, from_dev,
                     to_dev)
from ssdq import synth

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K = ssdq.Q4_0, ssdq.Q8_0, ssdq.Q4_K, ssdq.Q6_K


def run(dtype, w, x, out_dim, in_dim, batch=1, generic=False, w_dev=None):
    y = empty_dev(out_dim * batch, torch.float32)
    rc = ssdq.matvec(dtype, w_dev if w_dev is not None else to_dev(w), to_dev(x), y, out_dim,
                     in_dim, batch, generic=generic)
    return from_dev(y), rc


def reference(dtype, w, x, out_dim, in_dim, batch=1):
    x = np.asarray(x, np.float32).reshape(batch, -1)
    ys, ex = [], []
    for b in range(batch):
        ys.append(o.matvec(dtype, w, x[b], out_dim, in_dim, threads=16)[0])
        ex.append(o.matvec_exact(dtype, w, x[b], out_dim, in_dim))
    return np.concatenate(ys), np.concatenate(ex)


CONFIGS = [
    # (dtype, out_dim, in_dim, batch, label)
    (Q4_0, 4096, 4096, 1, "config1"),
    (Q4_0, 14336, 4096, 1, "north-star Q4_0"),
    (Q8_0, 11008, 4096, 1, "config2 B=1"),
    (Q8_0, 11008, 4096, 4, "config2 B=4"),
    (Q8_0, 11008, 4096, 8, "config2 B=8"),
    (Q4_K, 14336, 4096, 1, "config3 W_up"),
    (Q6_K, 4096, 14336, 1, "config3 W_down"),
]


@pytest.mark.parametrize("dtype,out_dim,in_dim,batch,label", CONFIGS)
def test_matvec_configs(dtype, out_dim, in_dim, batch, label):
    cfg = 1 if "config1" in label else 2 if "config2" in label else 3
    w = synth.quant_weights(dtype, out_dim, in_dim, synth.seed(cfg, 0))
    x = synth.normal_f32((batch, in_dim), synth.seed(cfg, 1 + batch))
    announce("matvec", label, ssdq.TYPE_NAMES[dtype], out_dim, in_dim, batch)
    y, rc = run(dtype, w, x, out_dim, in_dim, batch)
    ref, exact = reference(dtype, w, x, out_dim, in_dim, batch)
    assert rc == 0
    n = assert_close_attributed(y, ref, exact, label)
    print(f"{label}: {n} ill-conditioned outputs compared to the exact sum")


@pytest.mark.parametrize("dtype", ssdq.QUANT_TYPES)
def test_generic_kernel_matches(dtype):
    in_dim = 4096 if dtype != Q6_K else 14336 // 2
    w = synth.quant_weights(dtype, 300, in_dim, 41)
    x = synth.normal_f32((3, in_dim), 42)
    announce("matvec generic", ssdq.TYPE_NAMES[dtype])
    y, rc = run(dtype, w, x, 300, in_dim, 3, generic=True)
    ref, exact = reference(dtype, w, x, 300, in_dim, 3)
    assert rc == 0
    assert_close_attributed(y, ref, exact, "generic")


@pytest.mark.parametrize("dtype", ssdq.QUANT_TYPES)
def test_misaligned_weights_take_generic_path(dtype):
    out_dim, in_dim = 65, 1024
    w = synth.quant_weights(dtype, out_dim, in_dim, 43)
    buf = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda")
    buf[1:1 + w.size] = to_dev(w)
    x = synth.normal_f32(in_dim, 44)
    announce("matvec misaligned", ssdq.TYPE_NAMES[dtype])
    y, rc = run(dtype, None, x, out_dim, in_dim, 1, w_dev=buf[1:])
    ref, exact = reference(dtype, w, x, out_dim, in_dim)
    assert rc == 0
    assert_close_attributed(y, ref, exact, "misaligned")


ODD = [
    (Q4_0, 1, 32, 1), (Q4_0, 3, 96, 2), (Q4_0, 257, 4096 + 17, 3), (Q4_0, 70, 32 * 9, 1),
    (Q8_0, 5, 64, 5), (Q8_0, 129, 32 * 7, 7), (Q8_0, 64, 8192, 16), (Q8_0, 1000, 32 * 12, 6),
    (Q8_0, 17, 32 * 64, 21), (Q8_0, 7, 16, 4),  # the last: rows shorter than one block
    (Q8_0, 40, 32 * 2, 3), (Q8_0, 300, 4096, 2),
    (Q4_K, 1, 256, 1), (Q4_K, 33, 256 * 3, 6), (Q4_K, 200, 256 * 40 + 100, 2), (Q4_K, 64, 4096, 9),
    (Q6_K, 2, 256, 1), (Q6_K, 31, 256 * 5, 3), (Q6_K, 100, 256 * 7, 8),
]


@pytest.mark.parametrize("dtype,out_dim,in_dim,batch", ODD)
def test_ragged_shapes(dtype, out_dim, in_dim, batch):
    w = synth.quant_weights(dtype, out_dim, in_dim, 50 + out_dim)
    x = synth.normal_f32((batch, in_dim), 51 + in_dim)
    announce("matvec ragged", ssdq.TYPE_NAMES[dtype], out_dim, in_dim, batch)
    y, rc = run(dtype, w, x, out_dim, in_dim, batch)
    ref, exact = reference(dtype, w, x, out_dim, in_dim, batch)
    assert rc == 0
    assert_close_attributed(y, ref, exact, "ragged")


def test_q4_k_closed_form_all_scales():
    # 64 rows, row i uses 6-bit scales / mins (i + 7 sb) % 64 and (3 i + 11 sb + 5) % 64,
    # d = 1, dmin = 0.5, q = j % 16, x = 1 -> exact integers / halves
    rows = []
    want = []
    q = np.arange(256) % 16
    for i in range(64):
        s = (i + 7 * np.arange(8)) % 64
        m = (3 * i + 11 * np.arange(8) + 5) % 64
        rows.append(enc.enc_q4_k(enc.f16_bits(1.0), enc.f16_bits(0.5), s, m, q))
        want.append((s * q.reshape(8, 32).sum(1)).sum() - 0.5 * (m * 32).sum())
    w = np.concatenate(rows)
    announce("matvec q4_k closed form")
    y, _ = run(Q4_K, w, np.ones(256, np.float32), 64, 256)
    assert np.array_equal(y, np.array(want, np.float32))


def test_reference_known_answers_through_host_twin():
    # compute.rs:2347-2381 through the MetalCompute-style synchronous API
    with ssdq.Context() as ctx:
        blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), np.full(16, 0x88, np.uint8)])
        announce("host twin KAT")
        assert abs(ctx.matvec_quantized(blk, np.ones(32, np.float32), 1, 32, Q4_0)[0]) < 1e-5
        blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), np.ones(32, np.uint8)])
        assert abs(ctx.matvec_quantized(blk, np.ones(32, np.float32), 1, 32, Q8_0)[0] - 32.0) < 1e-3
        # a short weight buffer is an error, not a crash
        with pytest.raises(ssdq.SsdqError):
            ctx.matvec_quantized(blk[:20], np.ones(32, np.float32), 1, 32, Q8_0)
        # unsupported dtype -> zeros (compute.rs:672-675)
        y = ctx.matvec_quantized(np.zeros(64, np.uint8), np.ones(32, np.float32), 3, 32, 3)
        assert np.all(y == 0)
        # a config-sized call through the host twin
        w = synth.quant_weights(Q4_K, 1024, 4096, 61)
        x = synth.normal_f32(4096, 62)
        y = ctx.matvec_quantized(w, x, 1024, 4096, Q4_K)
        ref, exact = reference(Q4_K, w, x, 1024, 4096)
        assert_close_attributed(y, ref, exact, "host twin")


def test_unsupported_dtype_zero_fills_device():
    y = empty_dev(16, torch.float32)
    y.fill_(3.0)
    x = to_dev(np.ones(64, np.float32))
    announce("matvec unsupported")
    rc = ssdq.matvec(3, x, x, y, 16, 64)
    assert rc == ssdq.WARN_UNSUPPORTED_ZEROED and np.all(from_dev(y) == 0)


def test_repeat_is_deterministic():
    w = synth.quant_weights(Q4_K, 14336, 4096, 7)
    x = synth.normal_f32(4096, 8)
    wd = to_dev(w)
    announce("matvec determinism")
    a, _ = run(Q4_K, None, x, 14336, 4096, w_dev=wd)
    b, _ = run(Q4_K, None, x, 14336, 4096, w_dev=wd)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("dtype,batch", [(Q8_0, 4), (Q4_K, 4), (Q8_0, 1), (Q4_K, 1)])
def test_extreme_and_nonfinite_activations(dtype, batch):
    # row 0 normal; row 1 with one NaN (the reference's serial sum is NaN for
    # every output); row 2 with a whole 32-element block scaled by 1e30 and a
    # 1e3 outlier in another block; row 3 scaled to ~1e-30; row 4 scaled to
    # ~1e-35 (32-element groups whose largest value is below 2^-105, where
    # 2^(30 - e) as a factor would overflow); row 5 scaled to ~1e-37 (below
    # 2^-119, where the scale of the digit grid stops at 2^-149).  Batch 1
    # takes the rows one call at a time, batch 4 runs rows 0-3 as one batch and
    # rows 4 and 5 alone.  (x is
    # carried relative to the largest value of its 32-element block, with 30
    # bits: values more than ~9 orders below it are not.)
    out_dim, in_dim = 300, 4096
    w = synth.quant_weights(dtype, out_dim, in_dim, 71)
    x = synth.normal_f32((6, in_dim), 72)
    x[1, 1000] = np.nan
    x[2, 64:96] *= np.float32(1e30)
    x[2, 200] = np.float32(1e3)
    x[3] *= np.float32(1e-30)
    x[4] *= np.float32(1e-35)
    x[5] *= np.float32(1e-37)
    assert np.abs(x[4]).max() < 2.0 ** -105
    assert np.abs(x[5]).max() < 2.0 ** -119  # the digit grid's scale stops at 2^-149
    announce("matvec extreme activations", ssdq.TYPE_NAMES[dtype], batch)
    if batch == 4:
        y, rc = run(dtype, w, x[:4], out_dim, in_dim, 4)
        assert rc == 0
        rows = [y.reshape(4, out_dim)]
        for b in (4, 5):
            yb, rc = run(dtype, w, x[b], out_dim, in_dim, 1)
            assert rc == 0
            rows.append(yb.reshape(1, out_dim))
        y = np.concatenate(rows)
    else:
        rows = []
        for b in range(6):
            yb, rc = run(dtype, w, x[b], out_dim, in_dim, 1)
            assert rc == 0
            rows.append(yb)
        y = np.stack(rows)
    ref, exact = reference(dtype, w, x, out_dim, in_dim, 6)
    ref, exact = ref.reshape(6, out_dim), exact.reshape(6, out_dim)
    assert np.all(np.isnan(ref[1])) and np.all(np.isnan(y[1]))
    for b in (0, 2):
        assert_close_attributed(y[b], ref[b], exact[b], f"row {b}")
    # rows 3-5: relative agreement (the absolute 1e-4 term says nothing at
    # these magnitudes); the exact sums are double precision, so they hold the
    # 1e-35-scaled outputs (~1e-33, fp32 subnormal) without underflow
    for b in (3, 4, 5):
        assert np.all(np.isfinite(y[b])), f"row {b}: non-finite output"
        scale = np.abs(exact[b]).max()
        assert scale > 0
        assert np.all(np.abs(y[b] - exact[b]) <= 1e-3 * scale), f"row {b}"


Q8_MFMA = [  # (out_dim, in_dim, batch): Q8_0 batches of 2-8 on the matrix cores
    (11008, 4096, 2), (11008, 4096, 3), (11008, 4096, 5), (11008, 4096, 6), (11008, 4096, 7),
    (4097, 4096, 8), (1000, 2048, 3), (17, 1024, 5), (4096, 1024, 8), (16, 4096, 2), (300, 4096, 12),
    (20000, 4096, 4), (12289, 2048, 8),  # runs capped at 48 rows: more workgroups than CUs
]


@pytest.mark.parametrize("out_dim,in_dim,batch", Q8_MFMA)
def test_q8_0_small_batch_matrix_cores(out_dim, in_dim, batch):
    # ragged row groups (out_dim not a multiple of 16), every batch size 2-8,
    # K = 1024 / 2048 / 4096, and a batch of 12 (one chunk of 8 on the matrix
    # cores, then 4)
    w = synth.quant_weights(Q8_0, out_dim, in_dim, 800 + batch + out_dim)
    x = synth.normal_f32((batch, in_dim), 900 + batch)
    announce("q8_0 small batch", out_dim, in_dim, batch)
    y, rc = run(Q8_0, w, x, out_dim, in_dim, batch)
    assert rc == 0
    ref, exact = reference(Q8_0, w, x, out_dim, in_dim, batch)
    n = assert_close_attributed(y, ref, exact, f"q8_0 {out_dim}x{in_dim} B={batch}")
    # run-to-run bit identity (fixed summation order)
    y2, _ = run(Q8_0, w, x, out_dim, in_dim, batch)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def test_q8_0_small_batch_misaligned_x_takes_other_kernel():
    # x at a 4-byte offset cannot feed the 16-byte loads: the digit-plane kernel runs
    out_dim, in_dim, batch = 500, 4096, 4
    w = synth.quant_weights(Q8_0, out_dim, in_dim, 77)
    x = synth.normal_f32((batch, in_dim), 78)
    buf = torch.empty(batch * in_dim + 1, dtype=torch.float32, device="cuda")
    buf[1:].copy_(torch.from_numpy(x.ravel()).cuda())
    y = empty_dev(out_dim * batch, torch.float32)
    announce("q8_0 small batch misaligned")
    assert ssdq.matvec(Q8_0, to_dev(w), buf[1:], y, out_dim, in_dim, batch) == 0
    ref, exact = reference(Q8_0, w, x, out_dim, in_dim, batch)
    assert_close_attributed(from_dev(y), ref, exact, "q8_0 misaligned x")


LONG_ROWS = [  # batch-1 rows of 129-256 units (K slices summed in slice order)
    (Q4_K, 77, 256 * 36), (Q4_K, 1000, 256 * 64), (Q4_K, 4096, 14336),
    (Q4_0, 300, 64 * 144), (Q4_0, 64, 64 * 256), (Q8_0, 129, 64 * 192), (Q8_0, 4096, 14336),
    # whole rows beyond one round of workgroups: per-wave row streams, one slice
    (Q4_0, 40000, 2048), (Q4_K, 50000, 4096), (Q6_K, 60000, 2048), (Q8_0, 33333, 1024),
    (Q4_K, 40000, 2048),  # rows of 32 units through the LDS row copies: partial copies, dummy third copy
    (Q8_0, 50000, 2048),  # Q8_0 rows of 32 units through the LDS row copies (five 1 KB copies per row)
    (Q4_K, 50000, 6144),  # whole rows of 96 units, two units per lane through LDS (partial second unit)
]


@pytest.mark.parametrize("dtype,out_dim,in_dim", LONG_ROWS)
def test_batch1_long_rows(dtype, out_dim, in_dim):
    w = synth.quant_weights(dtype, out_dim, in_dim, 80 + out_dim)
    x = synth.normal_f32(in_dim, 81 + in_dim)
    announce("matvec long rows", ssdq.TYPE_NAMES[dtype], out_dim, in_dim)
    y, rc = run(dtype, w, x, out_dim, in_dim)
    assert rc == 0
    sel = np.arange(out_dim) if out_dim <= 1000 else np.r_[0:500, out_dim - 500:out_dim]
    rb = w.size // out_dim
    ref, exact = reference(dtype, w.reshape(out_dim, rb)[sel].ravel(), x, sel.size, in_dim)
    assert_close_attributed(y[sel], ref, exact, "long rows")
    y2, _ = run(dtype, w, x, out_dim, in_dim)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))  # fixed summation order


K_SLICED = [  # K-sliced rows: slice partials in the workspace, summed in slice order
    (Q4_K, 28672, 8192),   # LDS row slots of 3 KB, 2 slices of 2304 bytes
    (Q4_K, 4096, 14336),   # LDS row slots, 4 slices of 14 blocks, 64-row runs (12 row waves)
    (Q6_K, 4096, 14336),   # LDS row slots, 7 slices of 8 blocks, 113-row runs (8 row waves, two slots)
    (Q8_0, 4096, 28672),   # batch-1 kernel, 7 slices, interleaved row streams
    (Q4_0, 2000, 28800),   # 8 slices, partial last slice
    (Q6_K, 33, 14336),     # fewer rows than row streams
    (Q6_K, 128256, 4096),  # output-head shape: whole-row LDS streams (128 units per row), no slices
    (Q6_K, 20000, 8192),   # LDS row slots, 4 slices of 8 blocks (Q6_K head of an 8192-wide model)
    (Q4_K, 40000, 8704),   # LDS row slots, 3 slices of 12, 12 and 10 blocks (short last slice)
    # the row-slot K slices around their wave layouts (256 CUs, 4 slices: 64 runs)
    (Q4_K, 1030, 14336),   # 16-17 rows per run (ragged shares), two slots per wave
    (Q4_K, 5000, 14336),   # 78-79 rows per run, 12 row waves with one slot
    (Q4_K, 5200, 14336),   # 81-82 rows per run, 8 row waves with two slots
    (Q6_K, 9000, 14336),   # 250 rows per run (7 slices, 36 runs), clamped repeats after the last row
]


@pytest.mark.parametrize("dtype,out_dim,in_dim", K_SLICED)
def test_k_sliced_single_launch_repeats(dtype, out_dim, in_dim):
    """Three calls in a row agree bit for bit (the workspace's partials are
    rewritten by each call) and match the oracle."""
    w = synth.quant_weights(dtype, out_dim, in_dim, 90 + out_dim)
    x = synth.normal_f32(in_dim, 91 + in_dim)
    announce("k-sliced repeats", ssdq.TYPE_NAMES[dtype], out_dim, in_dim)
    w_dev = to_dev(w)
    ys = [run(dtype, None, x, out_dim, in_dim, w_dev=w_dev)[0] for _ in range(3)]
    for yk in ys[1:]:
        assert np.array_equal(ys[0].view(np.uint32), yk.view(np.uint32))
    sel = np.arange(out_dim) if out_dim <= 1000 else np.r_[0:300, out_dim // 2:out_dim // 2 + 100, out_dim - 300:out_dim]
    rb = w.size // out_dim
    ref, exact = reference(dtype, w.reshape(out_dim, rb)[sel].ravel(), x, sel.size, in_dim)
    assert_close_attributed(ys[0][sel], ref, exact, "k-sliced repeats")


ROW_SLOTS = [  # whole rows of 4096 through the LDS row slots (mv_b1r), at and around
    # the rows-per-CU thresholds of its two forms (256 CUs: 8, 24 and 80 rows per
    # CU, one round of the batch-1 kernel at 120): ragged workgroup shares,
    # clamped repeat rows after a wave's last, waves with one row more than others
    (Q4_K, 2048), (Q4_K, 2049), (Q4_K, 6143), (Q4_K, 6144), (Q4_K, 14335), (Q4_K, 20480),
    (Q4_K, 20481), (Q4_K, 30720), (Q4_0, 2051), (Q4_0, 11008), (Q4_0, 30719),
    (Q8_0, 2048), (Q8_0, 11009), (Q8_0, 28672),
]


@pytest.mark.parametrize("dtype,out_dim", ROW_SLOTS)
def test_batch1_row_slots(dtype, out_dim):
    in_dim = 4096
    w = synth.quant_weights(dtype, out_dim, in_dim, 1200 + out_dim)
    x = synth.normal_f32(in_dim, 1201 + out_dim)
    announce("matvec row slots", ssdq.TYPE_NAMES[dtype], out_dim, in_dim)
    wd = to_dev(w)
    y, rc = run(dtype, None, x, out_dim, in_dim, w_dev=wd)
    assert rc == 0
    # the first, middle and last rows, and every 97th row between
    sel = np.unique(np.r_[0:600, out_dim // 2 - 300:out_dim // 2 + 300, max(0, out_dim - 600):out_dim,
                          0:out_dim:97])
    rb = w.size // out_dim
    ref, exact = reference(dtype, w.reshape(out_dim, rb)[sel].ravel(), x, sel.size, in_dim)
    assert_close_attributed(y[sel], ref, exact, "row slots")
    y2, _ = run(dtype, None, x, out_dim, in_dim, w_dev=wd)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))  # fixed summation order
