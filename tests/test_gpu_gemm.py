"""Prefill GEMM parity (config 4): Y = X(bf16) W(Q4_K)^T against the per-token
matvec oracle (transformer.rs:166-196 -> matvec_q4_k_cpu, compute.rs:707-750)."""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, assert_close_attributed, empty_dev, from_dev, to_dev
from ssdq import synth

pytestmark = pytest.mark.gpu

LAYER = [  # Llama-3-8B decoder layer, (name, N, K)
    ("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
    ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336),
]


def gemm(w, xb, M, N, K):
    y = empty_dev(M * N, torch.float32)
    rc = ssdq.gemm_q4k_bf16(to_dev(w), to_dev(xb), y, M, N, K)
    return from_dev(y), rc


@pytest.mark.parametrize("name,N,K", LAYER)
def test_gemm_config4(name, N, K):
    M = 512
    w = synth.quant_weights(ssdq.Q4_K, N, K, synth.seed(4, LAYER.index((name, N, K))))
    xb = synth.f32_to_bf16_bits(synth.normal_f32((M, K), synth.seed(4, 8 + (K > 4096))))
    announce("gemm", name, M, N, K)
    y, rc = gemm(w, xb, M, N, K)
    assert rc == 0
    # every one of the 512 tokens is checked
    ref = o.gemm_q4k_bf16(w, xb, M, N, K, threads=16)
    exact = o.gemm_q4k_bf16(w, xb, M, N, K, threads=16, exact=True)
    n = assert_close_attributed(y, ref, exact, f"gemm {name}")
    print(f"gemm {name}: {n} ill-conditioned outputs compared to the exact sum")


def _extreme_rows(M, K, seed):
    """bf16 X at config-4 shapes: N(0, 1) rows, plus rows that leave fp16's
    range or its 2^26 window.  Returns the bf16 bits, the special rows, and the
    power of two each row was scaled by (1 for unscaled rows): scaling by a
    power of two commutes with the bf16 rounding, so row r's exact outputs are
    scale[r] times those of the unscaled row, and the tolerance's absolute term
    (1e-4 for unit-scale activations) is compared at that scale."""
    x = synth.normal_f32((M, K), seed)
    g = np.random.default_rng(seed + 1)
    scale = np.ones(M)
    r_spike, r_big, r_tiny, r_denorm, r_mixed, r_one_tiny = 3, 130, 257, 300, 389, 511
    cols = g.choice(K, 6, replace=False)
    x[r_spike, cols] = np.float32(1e5) * np.sign(g.standard_normal(6)).astype(np.float32)
    x[r_big] *= np.float32(2.0 ** 100)           # an all-large row (~1e30; fp16 max is 65504)
    scale[r_big] = 2.0 ** 100
    x[r_tiny] *= np.float32(2.0 ** -100)         # an all-tiny row (~1e-30, below fp16's subnormals)
    x[r_denorm] *= np.float32(2.0 ** -129)       # bf16 / fp32 subnormals (~1e-39)
    x[r_mixed, :K // 2] *= np.float32(2.0 ** 66)   # halves 40 orders of magnitude apart
    x[r_mixed, K // 2:] *= np.float32(2.0 ** -66)
    scale[r_mixed] = 2.0 ** 66
    x[r_one_tiny, 17] = np.float32(1e-30)        # a single tiny element in a normal row
    rows = dict(spike=r_spike, big=r_big, tiny=r_tiny, denorm=r_denorm, mixed=r_mixed, one_tiny=r_one_tiny)
    return synth.f32_to_bf16_bits(x), rows, scale


@pytest.mark.parametrize("name,N,K", [("q", 4096, 4096), ("gate", 14336, 4096), ("down", 4096, 14336)])
def test_gemm_extreme_rows(name, N, K):
    """Rows out of fp16's range (|x| from ~1e30 down to ~1e-39) at config-4
    shapes and weights.  Small rows are scaled into the fp16 window by a power of
    two per (row, super-block) and meet the same bar as N(0, 1) rows (tiny rows
    relative to their largest output); rows with values beyond 65504 (the 1e5
    spikes, the 2^100 and 2^66 rows) are recomputed in the reference's serial
    order and equal the oracle bit for bit, whatever the K split."""
    M = 512
    w = synth.quant_weights(ssdq.Q4_K, N, K, synth.seed(4, LAYER.index((name, N, K))))
    xb, rows, scale = _extreme_rows(M, K, 4242 + K)
    announce("gemm extreme rows", name, M, N, K)
    y, rc = gemm(w, xb, M, N, K)
    assert rc == 0
    ref = o.gemm_q4k_bf16(w, xb, M, N, K, threads=16).reshape(M, N)
    exact = o.gemm_q4k_bf16(w, xb, M, N, K, threads=16, exact=True).reshape(M, N)
    y = y.reshape(M, N)
    assert np.all(np.isfinite(ref)), "the oracle overflowed: the test rows are mis-sized"
    small = [rows["tiny"], rows["denorm"]]
    normal = np.setdiff1d(np.arange(M), small)
    sc = scale[normal][:, None]
    n = assert_close_attributed(y[normal] / sc, ref[normal] / sc, exact[normal] / sc, f"gemm extreme {name}")
    print(f"gemm extreme {name}: {n} ill-conditioned outputs compared to the exact sum")
    for r in small:
        top = np.abs(exact[r]).max()
        assert top > 0 and np.all(np.isfinite(y[r]))
        assert np.all(np.abs(y[r] - exact[r]) <= 1e-3 * top), f"row {r}"
    for r in (rows["spike"], rows["big"], rows["mixed"]):
        assert np.array_equal(y[r].view(np.uint32), ref[r].view(np.uint32)), f"row {r} not bit-exact"


@pytest.mark.parametrize("name,N,K", [("q", 4096, 4096), ("gate", 14336, 4096)])
def test_gemm_huge_and_nonfinite_rows(name, N, K):
    """±3e38 elements (bf16's top binade) next to N(0, 1) values in one
    super-block, rows of ±1e36, and NaN / infinity rows.  Weights are drawn with
    d, dmin ~ U[1e-5, 1e-4] so that the reference's fp32 products stay finite
    (|w| < 0.1).  A super-block whose range exceeds the fp16 window is recomputed
    in the reference's own order: those
    rows equal the oracle bit for bit (NaN payloads aside), whatever the K split."""
    M = 512
    g = np.random.default_rng(77 + N)
    w = synth.quant_weights(ssdq.Q4_K, N, K, 5151 + N)
    blk = w.reshape(-1, 144)
    for off in (0, 2):  # d, dmin ~ U[1e-5, 1e-4]
        blk[:, off:off + 2] = g.uniform(1e-5, 1e-4, blk.shape[0]).astype(np.float16).view(np.uint8).reshape(-1, 2)
    x = synth.normal_f32((M, K), 5252 + N)
    r_huge, r_huge2, r_big, r_nan, r_inf, r_ninf = 1, 140, 255, 300, 410, 500
    x[r_huge, [5, 1000, 3001]] = np.float32([3e38, -3e38, 3e38])
    x[r_huge2, 2048] = np.float32(-3.3e38)
    x[r_big] *= np.float32(2.0 ** 120)  # ~1.3e36
    scale = np.ones(M)
    scale[r_big] = 2.0 ** 120
    x[r_nan, 77] = np.nan
    x[r_inf, 1234] = np.inf
    x[r_ninf, [3, 9]] = np.float32([-np.inf, np.inf])
    xb = synth.f32_to_bf16_bits(x)
    announce("gemm huge / non-finite rows", name, M, N, K)
    y, rc = gemm(w, xb, M, N, K)
    assert rc == 0
    y = y.reshape(M, N)
    ref = o.gemm_q4k_bf16(w, xb, M, N, K, threads=16).reshape(M, N)
    exact = o.gemm_q4k_bf16(w, xb, M, N, K, threads=16, exact=True).reshape(M, N)
    nonfinite = [r_nan, r_inf, r_ninf]
    finite = np.setdiff1d(np.arange(M), nonfinite)
    assert np.all(np.isfinite(ref[finite])), "the oracle overflowed: the test rows are mis-sized"
    sc = scale[finite][:, None]  # the scaled row is compared at its scale
    assert_close_attributed(y[finite] / sc, ref[finite] / sc, exact[finite] / sc, f"gemm huge {name}")
    for r in nonfinite:
        assert np.array_equal(np.isnan(y[r]), np.isnan(ref[r])), f"row {r}: NaN pattern"
        fin = ~np.isnan(ref[r])
        assert np.array_equal(y[r][fin], ref[r][fin]), f"row {r}: infinities"
    # rows out of the fp16 window are recomputed in the reference's order: the
    # oracle's bits, with one K split (gate) or several (q: 4 splits, the
    # other splits contribute exact zeros)
    for r in (r_huge, r_huge2, r_inf):
        fin = ~np.isnan(ref[r])
        assert np.array_equal(y[r][fin].view(np.uint32), ref[r][fin].view(np.uint32)), f"row {r} not bit-exact"


def test_gemm_wide_dmin():
    """Super-blocks whose |dmin| is 1024 or more (|dmin * m| beyond fp16's
    largest finite value) in some columns, beside ordinary columns of the same
    waves: the matrix-core min term of those columns runs scaled by 2^-10 and
    meets the same bar against the reference's serial fp32 chain."""
    M, N, K = 192, 512, 2048
    g = np.random.default_rng(4711)
    w = synth.quant_weights(ssdq.Q4_K, N, K, 4712)
    blk = w.reshape(N, K // 256, 144)
    for n in g.choice(N, 40, replace=False):
        sbs = g.choice(K // 256, 3, replace=False)
        v = g.uniform(1024.0, 60000.0, 3) * g.choice([-1.0, 1.0], 3)
        blk[n, sbs, 2:4] = v.astype(np.float16).view(np.uint8).reshape(-1, 2)
    blk[7, 0, 2:4] = np.float16(1024.0).reshape(1).view(np.uint8)  # the boundary itself
    blk[8, 1, 2:4] = np.float16(1023.5).reshape(1).view(np.uint8)  # just below it
    xb = synth.f32_to_bf16_bits(synth.normal_f32((M, K), 4713))
    announce("gemm wide dmin", M, N, K)
    y, rc = gemm(w, xb, M, N, K)
    assert rc == 0
    ref = o.gemm_q4k_bf16(w, xb, M, N, K, threads=8)
    exact = o.gemm_q4k_bf16(w, xb, M, N, K, threads=8, exact=True)
    assert np.all(np.isfinite(ref))
    assert_close_attributed(y, ref, exact, "gemm wide dmin")


@pytest.mark.parametrize("M,N,K", [(1, 16, 256), (7, 33, 512), (100, 64, 1024), (513, 40, 256),
                                   (512, 1024, 5376)])  # 8 K splits of 2-3 super-blocks (odd and even)
def test_gemm_ragged(M, N, K):
    w = synth.quant_weights(ssdq.Q4_K, N, K, M + N)
    xb = synth.f32_to_bf16_bits(synth.normal_f32((M, K), K))
    announce("gemm ragged", M, N, K)
    y, rc = gemm(w, xb, M, N, K)
    ref = o.gemm_q4k_bf16(w, xb, M, N, K, threads=8)
    exact = o.gemm_q4k_bf16(w, xb, M, N, K, threads=8, exact=True)
    assert rc == 0
    assert_close_attributed(y, ref, exact, "gemm ragged")


def test_gemm_rejects_bad_k():
    t = empty_dev(1024, torch.float32)
    with pytest.raises(ssdq.SsdqError):
        ssdq.gemm_q4k_bf16(t, t, t, 4, 4, 300)


def test_gemm_misaligned_x_takes_fallback():
    # X at a 2-byte offset cannot feed 16-byte loads: the widen + matvec path runs
    M, N, K = 9, 48, 512
    w = synth.quant_weights(ssdq.Q4_K, N, K, 77)
    xb = synth.f32_to_bf16_bits(synth.normal_f32((M, K), 78))
    buf = torch.empty(M * K + 1, dtype=torch.int16, device="cuda")
    buf[1:].copy_(torch.from_numpy(xb.view(np.int16).ravel()).cuda())
    y = empty_dev(M * N, torch.float32)
    announce("gemm misaligned", M, N, K)
    assert ssdq.gemm_q4k_bf16(to_dev(w), buf[1:], y, M, N, K) == 0
    ref = o.gemm_q4k_bf16(w, xb, M, N, K, threads=8)
    exact = o.gemm_q4k_bf16(w, xb, M, N, K, threads=8, exact=True)
    assert_close_attributed(from_dev(y), ref, exact, "gemm misaligned")


def multi(ws, xb, M, ns, K, x_dev=None):
    ys = [empty_dev(M * n, torch.float32) for n in ns]
    rc = ssdq.gemm_q4k_bf16_multi([to_dev(w) for w in ws], x_dev if x_dev is not None else to_dev(xb), ys, M,
                                  list(ns), K)
    return [from_dev(y) for y in ys], rc


@pytest.mark.parametrize("names", [("q", "k", "v"), ("gate", "up")])
def test_gemm_multi_config4(names):
    # q/k/v (and gate/up) share X: one GEMM over the concatenated columns
    M = 512
    mats = [m for m in LAYER if m[0] in names]
    K = mats[0][2]
    ws = [synth.quant_weights(ssdq.Q4_K, N, K, synth.seed(4, LAYER.index(m))) for m in mats for N in [m[1]]]
    xb = synth.f32_to_bf16_bits(synth.normal_f32((M, K), synth.seed(4, 8)))
    announce("gemm multi", names, M, K)
    ys, rc = multi(ws, xb, M, [m[1] for m in mats], K)
    assert rc == 0
    for (name, N, _), w, y in zip(mats, ws, ys):  # all 512 tokens
        ref = o.gemm_q4k_bf16(w, xb, M, N, K, threads=16)
        exact = o.gemm_q4k_bf16(w, xb, M, N, K, threads=16, exact=True)
        assert_close_attributed(y, ref, exact, f"gemm multi {name}")


@pytest.mark.parametrize("M,ns,K", [(77, (100, 37, 300), 512), (130, (256, 64), 768), (5, (300,), 256),
                                    (300, (1, 2, 3), 256)])
def test_gemm_multi_ragged(M, ns, K):
    ws = [synth.quant_weights(ssdq.Q4_K, n, K, 900 + i) for i, n in enumerate(ns)]
    xb = synth.f32_to_bf16_bits(synth.normal_f32((M, K), 901))
    announce("gemm multi ragged", M, ns, K)
    ys, rc = multi(ws, xb, M, ns, K)
    assert rc == 0
    for n, w, y in zip(ns, ws, ys):
        ref = o.gemm_q4k_bf16(w, xb, M, n, K, threads=8)
        exact = o.gemm_q4k_bf16(w, xb, M, n, K, threads=8, exact=True)
        assert_close_attributed(y, ref, exact, f"gemm multi ragged n={n}")
        # the single-matrix entry point computes the same columns
        y1, rc1 = gemm(w, xb, M, n, K)
        assert rc1 == 0
        assert_close_attributed(y, y1.astype(np.float32), exact, "multi vs single")


def test_gemm_multi_misaligned_x_takes_fallback():
    M, K, ns = 9, 512, (48, 20)
    ws = [synth.quant_weights(ssdq.Q4_K, n, K, 70 + n) for n in ns]
    xb = synth.f32_to_bf16_bits(synth.normal_f32((M, K), 79))
    buf = torch.empty(M * K + 1, dtype=torch.int16, device="cuda")
    buf[1:].copy_(torch.from_numpy(xb.view(np.int16).ravel()).cuda())
    announce("gemm multi misaligned", M, ns, K)
    ys, rc = multi(ws, xb, M, ns, K, x_dev=buf[1:])
    assert rc == 0
    for n, w, y in zip(ns, ws, ys):
        ref = o.gemm_q4k_bf16(w, xb, M, n, K, threads=8)
        exact = o.gemm_q4k_bf16(w, xb, M, n, K, threads=8, exact=True)
        assert_close_attributed(y, ref, exact, "gemm multi misaligned")


def test_gemm_multi_rejects_bad_arguments():
    t = empty_dev(4096, torch.float32)
    with pytest.raises(ssdq.SsdqError):  # four matrices
        ssdq.gemm_q4k_bf16_multi([t] * 4, t, [t] * 4, 4, [4] * 4, 256)
    with pytest.raises(ssdq.SsdqError):  # an empty matrix
        ssdq.gemm_q4k_bf16_multi([t, t], t, [t, t], 4, [4, 0], 256)
    with pytest.raises(ssdq.SsdqError):  # K not a multiple of 256
        ssdq.gemm_q4k_bf16_multi([t], t, [t], 4, [4], 300)
