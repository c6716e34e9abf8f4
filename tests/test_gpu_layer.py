"""Decode-layer ops on quantized weights, through the C ABI: QKV projection +
RoPE (fused_qkv_rope_f32_cpu, src/metal/compute.rs:509-534), SwiGLU gate/up
(src/inference/feed_forward.rs:28-40), RMSNorm + output head
(fused_rmsnorm_linear_f32_cpu, compute.rs:557-578) and the post-attention
residual + RMSNorm (fused_post_attn_norm_f32_cpu, compute.rs:536-555), each
with the projections through matvec_quantized_cpu.  Shapes are Llama-3-8B's
(n_embd 4096, 32 query / 8 KV heads of 128, n_ff 14336, vocab 128256) plus
cases that take the unfused path (mixed or extra types, rows of 80 units, odd
row counts) and other head counts and FFN widths for the fused launches.

Tolerance: the projections are held to |gpu - ref| <= 1e-4 + 1e-3 |ref| (with
the exact-sum substitution of helpers.assert_close_attributed).  RoPE and
SwiGLU combine two projections, and a small output can come from large inputs
(a rotated pair near cancellation; silu(g) ~ 100 times u ~ 0.007), so their
outputs are held to that tolerance propagated through the epilogue, against
the composition in double precision over exact projections:
  RoPE    |d o| <= tol(o) + |cos| tol(a0) + |sin| tol(a1)
  SwiGLU  |d h| <= tol(h) + |silu(g)| tol(u) + |silu'(g) u| tol(g)."""
import math

import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import (announce, assert_close, assert_close_attributed, assert_propagated, empty_dev, from_dev,
                     rope_bound, rope_double, swiglu_propagated, to_dev, tol)
from ssdq import synth

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0, Q4_0, Q5_K = ssdq.Q4_K, ssdq.Q6_K, ssdq.Q8_0, ssdq.Q4_0, ssdq.Q5_K


QKV = [
    # dtypes (q, k, v), n_embd, head_dim, position, theta, query heads, KV heads
    ((Q4_K, Q4_K, Q4_K), 4096, 128, 4000, 500000.0, 32, 8),   # fused
    ((Q6_K, Q6_K, Q6_K), 4096, 128, 31999, 500000.0, 32, 8),  # fused, two units per lane
    ((Q8_0, Q8_0, Q8_0), 4096, 128, 1, 10000.0, 32, 8),       # fused
    ((Q4_K, Q4_K, Q6_K), 4096, 128, 77, 500000.0, 32, 8),     # mixed types: separate launches
    ((Q5_K, Q5_K, Q5_K), 4096, 128, 12345, 500000.0, 32, 8),  # an extra type: separate launches
    ((Q4_K, Q4_K, Q4_K), 4096, 0, 5, 10000.0, 32, 8),         # no rotation (fused_qkv_f32)
    ((Q4_K, Q4_K, Q4_K), 5120, 128, 5, 10000.0, 32, 8),       # 80 units per row: separate launches
    # fused, other head counts: (30, 6) is 2688 row pairs (10 or 11 per CU on
    # 256 CUs), (10, 2) 896 pairs (3 or 4), (2, 1) 256 pairs (1 per CU), (1, 1)
    # 128 pairs (fewer than the CUs: the kernel of register rows)
    ((Q4_K, Q4_K, Q4_K), 4096, 128, 1210, 500000.0, 30, 6),
    ((Q8_0, Q8_0, Q8_0), 4096, 128, 1210, 500000.0, 30, 6),
    ((Q4_0, Q4_0, Q4_0), 4096, 128, 1070, 500000.0, 10, 2),
    ((Q4_K, Q4_K, Q4_K), 4096, 128, 1014, 500000.0, 2, 1),
    ((Q4_K, Q4_K, Q4_K), 4096, 128, 1007, 500000.0, 1, 1),
]


@pytest.mark.parametrize("dts,n_embd,head_dim,position,theta,nh,nkv", QKV)
def test_qkv_rope(dts, n_embd, head_dim, position, theta, nh, nkv):
    q_dim, kv_dim = nh * 128, nkv * 128
    ws = [synth.quant_weights(dt, rows, n_embd, 700 + i) for i, (dt, rows) in
          enumerate(zip(dts, (q_dim, kv_dim, kv_dim)))]
    x = synth.normal_f32(n_embd, 701)
    q, k, v = empty_dev(q_dim, torch.float32), empty_dev(kv_dim, torch.float32), empty_dev(kv_dim, torch.float32)
    announce("qkv rope", [ssdq.TYPE_NAMES[d] for d in dts], n_embd, head_dim, position, nh, nkv)
    rc = ssdq.qkv_rope(dts, [to_dev(w) for w in ws], to_dev(x), q, k, v, q_dim, kv_dim, n_embd, head_dim,
                       position, theta)
    assert rc == 0
    rq, rk, rv = o.qkv_rope(dts[0], ws[0], dts[1], ws[1], dts[2], ws[2], x, q_dim, kv_dim, n_embd, head_dim,
                            position, theta)
    for name, got, ref, w, dt, rows, rot in (("q", q, rq, ws[0], dts[0], q_dim, True),
                                             ("k", k, rk, ws[1], dts[1], kv_dim, True),
                                             ("v", v, rv, ws[2], dts[2], kv_dim, False)):
        ex = o.matvec_exact(dt, w, x, rows, n_embd)
        if rot and head_dim:
            bound = rope_bound(ex, head_dim, position, theta)
            assert_propagated(from_dev(got), rope_double(ex, head_dim, position, theta), bound,
                              f"{name} {ssdq.TYPE_NAMES[dt]}")
        else:
            assert_close_attributed(from_dev(got), ref, ex, f"{name} {ssdq.TYPE_NAMES[dt]}")


# n_ff 14336 is 56 row pairs per CU on 256 CUs; 14000 is 54 or 55, 300 is 1
# or 2, 200 fewer than the CUs (the kernel of register rows)
SWIGLU = [(Q4_K, 4096, 14336), (Q6_K, 4096, 14336), (Q4_0, 4096, 14336), (Q8_0, 4096, 14336),
          (Q5_K, 4096, 14336), (Q4_K, 5120, 14336), (Q4_K, 4096, 14000), (Q4_0, 4096, 300), (Q4_K, 4096, 200)]


@pytest.mark.parametrize("dtype,n_embd,n_ff", SWIGLU)
def test_swiglu(dtype, n_embd, n_ff):
    wg = synth.quant_weights(dtype, n_ff, n_embd, 800)
    wu = synth.quant_weights(dtype, n_ff, n_embd, 801)
    x = synth.normal_f32(n_embd, 802)
    h = empty_dev(n_ff, torch.float32)
    announce("swiglu", ssdq.TYPE_NAMES[dtype], n_embd, n_ff)
    assert ssdq.swiglu(dtype, to_dev(wg), to_dev(wu), to_dev(x), h, n_ff, n_embd) == 0
    ref = o.swiglu(dtype, wg, wu, x, n_ff, n_embd)
    g = o.matvec_exact(dtype, wg, x, n_ff, n_embd)
    u = o.matvec_exact(dtype, wu, x, n_ff, n_embd)
    ex, extra = swiglu_propagated(g, u)
    assert_propagated(from_dev(h), ex, extra, "swiglu")
    # and every output within the plain tolerance of the fp32 reference, except
    # where the reference's own chain is more than half a tolerance from the
    # exact composition
    assert_close_attributed(from_dev(h), ref, ex, "swiglu")


HEAD = [
    (Q6_K, 128256, 4096),  # Llama-3-8B output head, fused
    (Q4_K, 128256, 4096),
    (Q8_0, 32000, 4096),
    (Q4_K, 1001, 4096),    # odd row count (the norm-only kernel takes any)
    (Q5_K, 4096, 4096),    # an extra type: norm kernel + matvec
]


@pytest.mark.parametrize("dtype,vocab,n_embd", HEAD)
def test_rmsnorm_output_head(dtype, vocab, n_embd):
    w = synth.quant_weights(dtype, vocab, n_embd, 900)
    x = synth.normal_f32(n_embd, 901) * np.float32(3.0)
    g = (0.5 + synth.rng(902).random(n_embd)).astype(np.float32)
    y = empty_dev(vocab, torch.float32)
    announce("rmsnorm output head", ssdq.TYPE_NAMES[dtype], vocab, n_embd)
    assert ssdq.rmsnorm_matvec(dtype, to_dev(w), to_dev(x), to_dev(g), 1e-5, y, vocab, n_embd) == 0
    ref, rc = o.fused_rmsnorm_linear(dtype, w, x, g, vocab, n_embd)
    assert rc == 0
    inv = 1.0 / math.sqrt(float((x.astype(np.float64) ** 2).sum()) / n_embd + 1e-5)
    xn = (x.astype(np.float64) * inv * g).astype(np.float32)
    ex = o.matvec_exact(dtype, w, xn, vocab, n_embd)
    got = from_dev(y)
    # Outputs outside the tolerance of both the fp32 reference and the exact sum
    # are near-cancellations (|y| << sum |w x|).  The batch-1 kernel carries x
    # with 31 significant bits per 32-element group (x * norm_w rounded once in
    # fp32, then to the group's digit grid), so such an output may differ from
    # the exact sum by up to sum_e |w_e| (2^-31 max_group |x'| + 2^-24 |x'_e|).
    bad = np.flatnonzero((np.abs(got - ref) > tol(ref)) & (np.abs(got - ex) > tol(ex)))
    assert bad.size <= max(1, vocab // 10000), f"{bad.size} outputs outside tolerance"
    rb = len(w) // vocab
    xg = np.abs(xn.astype(np.float64))
    gmax = np.repeat(xg.reshape(-1, 32).max(axis=1), 32)
    for i in bad:
        e, rc = o.matvec_elements(dtype, w[i * rb:(i + 1) * rb], 1, n_embd)
        allow = tol(ex[i]) + float((np.abs(e[0].astype(np.float64)) * (gmax * 2.0 ** -31 + xg * 2.0 ** -24)).sum())
        assert abs(got[i] - ex[i]) <= allow, (i, got[i], ex[i], allow)
    print(f"{bad.size} near-cancelled outputs checked against the x-representation bound")


@pytest.mark.parametrize("n,with_res,inplace", [(4096, True, False), (4096, False, False), (5120, True, True),
                                                 (7, True, False)])
def test_rmsnorm(n, with_res, inplace):
    g = np.random.default_rng(n)
    x = g.standard_normal(n).astype(np.float32)
    res = g.standard_normal(n).astype(np.float32) if with_res else np.zeros(n, np.float32)
    w = (0.5 + g.random(n)).astype(np.float32)
    xd = to_dev(x)
    out = xd if inplace else empty_dev(n, torch.float32)
    hid = empty_dev(n, torch.float32)
    announce("rmsnorm", n, with_res, inplace)
    assert ssdq.rmsnorm(xd, to_dev(res) if with_res else None, to_dev(w), 1e-5, hid, out, n) == 0
    h_ref, o_ref = o.fused_post_attn_norm(x, res, w, 1e-5)
    assert_close(from_dev(hid), h_ref, "hidden")
    assert_close(from_dev(out), o_ref, "normalized")


def test_layer_ops_reject_bad_shapes():
    z = empty_dev(64, torch.float32)
    with pytest.raises(ssdq.SsdqError):  # odd q_dim
        ssdq.qkv_rope((Q4_K,) * 3, (z, z, z), z, z, z, z, 3, 2, 256, 0, 0, 1.0)
    with pytest.raises(ssdq.SsdqError):  # head_dim not dividing
        ssdq.qkv_rope((Q4_K,) * 3, (z, z, z), z, z, z, z, 4096, 1024, 256, 96, 0, 1.0)
