"""Committed golden fixtures (tests/golden/golden.json, written by
tests/golden/make_golden.py): the reference's known answers, small vectors of
every op, and digests of the full-size bit-exact outputs.  CPU tests pin the
oracle to them; GPU tests hold the device path to them."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, assert_close, empty_dev, from_dev, to_dev
from ssdq import synth

G = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))


def f32(bits_list):
    return np.asarray(bits_list, np.uint32).view(np.float32)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ------------------------------------------------------------------- CPU
@pytest.mark.parametrize("k", G["kats"], ids=lambda k: k["name"])
def test_oracle_reference_kats(k):
    w = np.frombuffer(bytes.fromhex(k["w_hex"]), np.uint8)
    y, _ = o.matvec(k["dtype"], w, np.asarray(k["x"], np.float32), k["out_dim"], k["in_dim"])
    assert np.all(np.abs(y - np.asarray(k["y"])) < k["abs_tol"])


@pytest.mark.parametrize("c", G["matvec"], ids=lambda c: c["name"])
def test_oracle_small_vectors(c):
    w = np.frombuffer(bytes.fromhex(c["w_hex"]), np.uint8)
    x = f32(c["x_bits"])
    deq, _ = o.dequantize(c["dtype"], w, c["out_dim"] * c["in_dim"])
    y, _ = o.matvec(c["dtype"], w, x, c["out_dim"], c["in_dim"])
    assert deq.view(np.uint32).tolist() == c["dequant_bits"]
    assert y.view(np.uint32).tolist() == c["y_bits"]


def test_oracle_int8_rows():
    c = G["int8"]
    data = f32(c["data_bits"])
    codes, scales = o.quantize_rows(data, c["n_rows"], c["dim"])
    assert codes.astype(int).tolist() == c["codes"]
    assert scales.view(np.uint32).tolist() == c["scale_bits"]
    assert o.dequantize_rows(codes, scales, c["n_rows"], c["dim"]).view(np.uint32).tolist() == c["dequant_bits"]


def _attn_inputs(c):
    return (f32(c["q_bits"]), np.asarray(c["k_codes"], np.int8), f32(c["k_scale_bits"]),
            np.asarray(c["v_codes"], np.int8), f32(c["v_scale_bits"]),
            np.asarray(c["block_tables"], np.int32).reshape(c["n_seq"], -1),
            np.asarray(c["ctx_lens"], np.int32))


def test_oracle_paged_attention():
    c = G["paged_attention"]
    q, kc, ks, vc, vs, tables, ctx = _attn_inputs(c)
    out = o.paged_attention_int8(q, kc, ks, vc, vs, tables, ctx, c["n_seq"], c["n_head"],
                                 c["n_head_kv"], c["head_dim"], c["block_size"],
                                 c["max_blocks_per_seq"])
    assert out.view(np.uint32).tolist() == c["out_bits"]


def test_synthetic_inputs_are_stable():
    # the full-size digests below assume the seeded generator is unchanged
    d = G["digests"][0]
    w = synth.quant_weights(d["dtype"], d["rows"], d["cols"], d["seed"])
    assert sha(w) == d["input_sha256"]


# ------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("c", G["kats"] + G["matvec"], ids=lambda c: c["name"])
def test_gpu_small_vectors(c):
    w = np.frombuffer(bytes.fromhex(c["w_hex"]), np.uint8).copy()
    x = np.asarray(c["x"], np.float32) if "x" in c else f32(c["x_bits"])
    announce("golden matvec", c["name"])
    y = empty_dev(c["out_dim"], torch.float32)
    ssdq.matvec(c["dtype"], to_dev(w), to_dev(x), y, c["out_dim"], c["in_dim"])
    got = from_dev(y)
    if "y_bits" in c:
        assert_close(got, f32(c["y_bits"]), "golden matvec")
        out = empty_dev(c["out_dim"] * c["in_dim"], torch.float32)
        ssdq.dequant(c["dtype"], to_dev(w), c["out_dim"] * c["in_dim"], out)
        assert from_dev(out).view(np.uint32).tolist() == c["dequant_bits"]
    else:
        assert np.all(np.abs(got - np.asarray(c["y"])) < c["abs_tol"])


@pytest.mark.gpu
def test_gpu_int8_rows():
    c = G["int8"]
    n = c["n_rows"] * c["dim"]
    codes = torch.empty(n, dtype=torch.int8, device="cuda")
    scales = empty_dev(c["n_rows"], torch.float32)
    announce("golden int8")
    ssdq.kv_quantize_rows(to_dev(f32(c["data_bits"])), codes, scales, c["n_rows"], c["dim"])
    assert from_dev(codes).astype(int).tolist() == c["codes"]
    assert from_dev(scales).view(np.uint32).tolist() == c["scale_bits"]


@pytest.mark.gpu
def test_gpu_paged_attention():
    c = G["paged_attention"]
    q, kc, ks, vc, vs, tables, ctx = _attn_inputs(c)
    out = empty_dev(q.size, torch.float32)
    announce("golden paged attention")
    ssdq.paged_attention_int8(to_dev(q), to_dev(kc), to_dev(ks), to_dev(vc), to_dev(vs),
                              to_dev(tables), to_dev(ctx), out, c["n_seq"], c["n_head"],
                              c["n_head_kv"], c["head_dim"], c["block_size"],
                              c["max_blocks_per_seq"], int(ctx.max()))
    assert_close(from_dev(out), f32(c["out_bits"]), "golden attention")


@pytest.mark.gpu
@pytest.mark.parametrize("d", G["digests"], ids=lambda d: d["what"])
def test_gpu_full_size_dequant_digest(d):
    w = synth.quant_weights(d["dtype"], d["rows"], d["cols"], d["seed"])
    assert sha(w) == d["input_sha256"]
    n = d["rows"] * d["cols"]
    out = empty_dev(n, torch.float32)
    announce("golden digest", d["what"])
    ssdq.dequant(d["dtype"], to_dev(w), n, out)
    assert sha(from_dev(out)) == d["output_sha256"]
