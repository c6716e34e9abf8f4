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
    # the device computes all 512 tokens; the oracle checks a 96-token sample
    # (first, middle and last tiles) to keep the CPU side to seconds
    sel = np.r_[0:32, 240:272, 480:512]
    xs = xb.reshape(M, K)[sel]
    ref = o.gemm_q4k_bf16(w, xs, sel.size, N, K, threads=16)
    exact = o.gemm_q4k_bf16(w, xs, sel.size, N, K, threads=16, exact=True)
    n = assert_close_attributed(y.reshape(M, N)[sel], ref, exact, f"gemm {name}")
    print(f"gemm {name}: {n} ill-conditioned outputs compared to the exact sum")


@pytest.mark.parametrize("M,N,K", [(1, 16, 256), (7, 33, 512), (100, 64, 1024), (513, 40, 256)])
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
    sel = np.r_[0:16, 250:266, 496:512]
    xs = xb.reshape(M, K)[sel]
    for (name, N, _), w, y in zip(mats, ws, ys):
        ref = o.gemm_q4k_bf16(w, xs, sel.size, N, K, threads=16)
        exact = o.gemm_q4k_bf16(w, xs, sel.size, N, K, threads=16, exact=True)
        assert_close_attributed(y.reshape(M, N)[sel], ref, exact, f"gemm multi {name}")


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
