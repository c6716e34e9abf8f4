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
