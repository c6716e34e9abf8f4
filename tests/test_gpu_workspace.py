"""The library's per-stream workspace under HIP graph capture.

A graph captured on a stream keeps the workspace address it saw.  A later,
larger eager call on the same stream grows the workspace; the old buffer must
stay valid (it is retired, not freed), so replays of the graph still read and
write live memory and still produce the oracle's result.  Tolerance: the
matvec bar, |gpu - ref| <= 1e-4 + 1e-3 |ref| (with the exact-sum substitution
of helpers.assert_close_attributed).
"""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, assert_close_attributed, to_dev
from ssdq import synth

pytestmark = pytest.mark.gpu


def test_graph_replay_after_workspace_growth():
    dev = torch.device("cuda")
    side = torch.cuda.Stream()
    # K-sliced Q4_K matvec (4096 x 14336): its slice partials live in the
    # workspace, summed by a second kernel
    out_dim, in_dim = 4096, 14336
    w = synth.quant_weights(ssdq.Q4_K, out_dim, in_dim, 901)
    x = synth.normal_f32(in_dim, 902)
    wd, xd = to_dev(w), to_dev(x)
    yd = torch.empty(out_dim, dtype=torch.float32, device=dev)
    ref = o.matvec(ssdq.Q4_K, w, x, out_dim, in_dim, threads=16)[0]
    exact = o.matvec_exact(ssdq.Q4_K, w, x, out_dim, in_dim)

    announce("workspace: eager warm-up and capture of a K-sliced matvec")
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        ssdq.matvec(ssdq.Q4_K, wd, xd, yd, out_dim, in_dim, stream=side)
    side.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        ssdq.matvec(ssdq.Q4_K, wd, xd, yd, out_dim, in_dim, stream=side)
    torch.cuda.synchronize()

    # a larger eager call on the same stream: the prefill GEMM's prepared X
    # (512 x 4096 fp16 plus sums, ~4 MB) outgrows the matvec's partials
    announce("workspace: larger eager GEMM on the captured stream")
    M, N, K = 512, 1024, 4096
    gw = synth.quant_weights(ssdq.Q4_K, N, K, 903)
    gx = synth.f32_to_bf16_bits(synth.normal_f32((M, K), 904))
    gy = torch.empty(M * N, dtype=torch.float32, device=dev)
    with torch.cuda.stream(side):
        ssdq.gemm_q4k_bf16(to_dev(gw), to_dev(gx), gy, M, N, K, stream=side)
    side.synchronize()

    # replays, with eager work and synchronizations between them
    for rep in range(4):
        announce("workspace: graph replay", rep)
        yd.fill_(np.nan)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = yd.cpu().numpy()
        assert_close_attributed(got, ref, exact, f"replay {rep}")
        # unrelated eager work on the side stream between replays
        with torch.cuda.stream(side):
            ssdq.matvec(ssdq.Q4_K, wd, xd, torch.empty_like(yd), out_dim, in_dim, stream=side)
        side.synchronize()

    # a reservation larger than anything so far also leaves the graph valid
    announce("workspace: reserve, then replay")
    ssdq.reserve_workspace(64 << 20, stream=side)
    yd.fill_(np.nan)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert_close_attributed(yd.cpu().numpy(), ref, exact, "after reserve")
    del g
    torch.cuda.synchronize()
    ssdq.release_workspaces()
