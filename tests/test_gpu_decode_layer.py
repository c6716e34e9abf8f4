"""One decoder layer for one token from device-resident GGUF weights
(ssdq_weights_* + ssdq_decode_layer_dev), against the oracle's composition of
the same steps: the per-layer body of forward_pass
(src/inference/transformer.rs:319-397) with multi_head_attention_fused_rope
(src/inference/attention.rs:172-240) over the paged INT8 KV cache and the
dense SwiGLU FFN (feed_forward.rs:16-71).  Tensors are uploaded once under
their GGUF names (the replacement of SsdStreamer::load_layer,
src/ssd/streamer.rs:43-66).

Each step's output is read back from the layer's scratch regions and checked
against the oracle run on the device's own input to that step, at that step's
bar:
  norms, attention             |gpu - ref| <= 1e-4 + 1e-3 |ref|
  projections (o, down)        the same, with the exact-sum substitution
  q / k (RoPE), SwiGLU         that bar propagated through the epilogue
  KV pool row, residual adds   bit-exact
Then the whole layer, oracle composition from the same input hidden state,
end to end.  The layer output is hidden + Wo a + W_down h, and an output can
be a near-cancellation of terms tens of times larger, so it is held to a bar
relative to the magnitude of the terms summed into it, S = |hidden| +
|Wo| |a| + |W_down| |h| (|W| the dequantized elements' magnitudes, a and h
the oracle's):
  |gpu - ref| <= 1e-4 + 1e-4 S
A K-term fp32 sum carries about sqrt(K) 2^-24 of its term scale in rounding
(7e-6 at K = 14336); the layer chains a few such sums on each side.  A wiring
mistake -- a wrong buffer, head or slot -- fails the step checks above and
moves outputs by O(that scale).  A second token at the next position reads
the first token's appended row through the block table."""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import (ATOL, announce, assert_close, assert_close_attributed, assert_propagated, bits_equal,
                     from_dev, rope_bound, rope_double, swiglu_propagated, to_dev)
from ssdq import synth

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0, Q4_0, Q5_K, F32, F16 = ssdq.Q4_K, ssdq.Q6_K, ssdq.Q8_0, ssdq.Q4_0, ssdq.Q5_K, ssdq.F32, ssdq.F16
EPS = 1e-5
BLOCK = 16
E2E_RTOL = 1e-4  # end-to-end bar, relative to the outputs' term scale


class Layer:
    """Synthetic weights of one layer: {suffix: (dtype, dims, raw)}."""

    def __init__(self, n_embd, n_head, n_kv, hd, n_ff, types, seed, norm_type=F32, drop=()):
        self.n_embd, self.n_head, self.n_kv, self.hd, self.n_ff = n_embd, n_head, n_kv, hd, n_ff
        # zero-mean blocks (a random sign per block), scaled so that each
        # projection maps O(1) inputs to O(1) outputs
        self.t = synth.decoder_layer(n_embd, n_head, n_kv, hd, n_ff, types, seed)
        g = synth.rng(seed + 50)
        for name in ("attn_norm", "ffn_norm"):
            w = (0.5 + g.random(n_embd)).astype(np.float32)
            if norm_type == F16:
                w16 = w.astype(np.float16)
                self.t[name] = (F16, (n_embd,), w16.view(np.uint8), w16.astype(np.float32))
            else:
                self.t[name] = (F32, (n_embd,), w.view(np.uint8), w)
        for name in drop:
            del self.t[name]

    def upload(self, store, layer):
        tensors = [(f"blk.{layer}.{k}.weight", v[0], v[1], v[2]) for k, v in self.t.items()]
        return store.load_layer(tensors, layer)

    def w(self, name):
        return self.t[name][2]

    def dt(self, name):
        return self.t[name][0]

    def norm(self, name):
        return self.t[name][3] if name in self.t else None

    def has(self, *names):
        return all(n in self.t for n in names)


class Pool:
    """A paged INT8 pool holding `ctx` earlier tokens of one sequence."""

    def __init__(self, kv_dim, ctx, max_blocks, n_phys, kv_rms, seed):
        g = synth.rng(seed)
        self.kv_dim, self.max_blocks = kv_dim, max_blocks
        self.table = g.permutation(n_phys)[:max_blocks].astype(np.int32)
        rows = n_phys * BLOCK
        self.kc = np.zeros(rows * kv_dim, np.int8)
        self.vc = np.zeros(rows * kv_dim, np.int8)
        self.ks = np.zeros(rows, np.float32)
        self.vs = np.zeros(rows, np.float32)
        k = (g.standard_normal((ctx, kv_dim)) * kv_rms[0]).astype(np.float32)
        v = (g.standard_normal((ctx, kv_dim)) * kv_rms[1]).astype(np.float32)
        for p in range(ctx):
            self.store(p, k[p], v[p])
        self.dev = None

    def upload(self):
        self.dev = [to_dev(a) for a in (self.kc, self.ks, self.vc, self.vs)]
        return self

    def slot(self, pos):
        return int(self.table[pos // BLOCK]) * BLOCK + pos % BLOCK

    def store(self, pos, k, v):
        r = self.slot(pos)
        kc, ks = o.quantize_rows(k, 1, self.kv_dim)
        vc, vs = o.quantize_rows(v, 1, self.kv_dim)
        self.kc[r * self.kv_dim:(r + 1) * self.kv_dim] = kc
        self.vc[r * self.kv_dim:(r + 1) * self.kv_dim] = vc
        self.ks[r], self.vs[r] = ks[0], vs[0]

    def from_device(self):
        return [from_dev(t) for t in self.dev]


def oracle_layer(L, hidden, pos, pool, theta, threads=16):
    """The oracle's composition of the layer, from `hidden`; appends this
    token's K/V to `pool` (host arrays) and returns (hidden out, steps)."""
    n_embd, q_dim, kv_dim = L.n_embd, L.n_head * L.hd, L.n_kv * L.hd
    st = {}
    st["attn_in"] = o.rmsnorm(hidden, L.norm("attn_norm"), EPS) if L.has("attn_norm") else hidden.copy()
    if not L.has("attn_q", "attn_k", "attn_v", "attn_output"):
        return hidden.copy(), st
    q, k, v = o.qkv_rope(L.dt("attn_q"), L.w("attn_q"), L.dt("attn_k"), L.w("attn_k"), L.dt("attn_v"),
                         L.w("attn_v"), st["attn_in"], q_dim, kv_dim, n_embd, L.hd, pos, theta)
    st["q"], st["k"], st["v"] = q, k, v
    pool.store(pos, k, v)
    st["attn"] = o.paged_attention_int8(q, pool.kc, pool.ks, pool.vc, pool.vs, pool.table, np.array([pos + 1]),
                                        1, L.n_head, L.n_kv, L.hd, BLOCK, pool.max_blocks, threads=threads)
    st["attn_out"] = o.matvec(L.dt("attn_output"), L.w("attn_output"), st["attn"], n_embd, q_dim,
                              threads=threads)[0]
    if L.has("ffn_norm"):
        h, st["ffn_in"] = o.fused_post_attn_norm(hidden, st["attn_out"], L.norm("ffn_norm"), EPS)
        fin = st["ffn_in"]
    else:
        h = (hidden + st["attn_out"]).astype(np.float32)
        fin = h
    if L.has("ffn_gate", "ffn_up", "ffn_down"):
        g, _ = o.matvec(L.dt("ffn_gate"), L.w("ffn_gate"), fin, L.n_ff, n_embd, threads=threads)
        u, _ = o.matvec(L.dt("ffn_up"), L.w("ffn_up"), fin, L.n_ff, n_embd, threads=threads)
        st["ffn_h"] = (o.silu(g) * u).astype(np.float32)
        st["ffn_out"] = o.matvec(L.dt("ffn_down"), L.w("ffn_down"), st["ffn_h"], n_embd, L.n_ff,
                                 threads=threads)[0]
        h = (h + st["ffn_out"]).astype(np.float32)
    return h, st


def run_gpu_layer(store, layer, cfg, hidden, pos, pool, scratch, offs, steps):
    hd = to_dev(hidden)
    bt = to_dev(pool.table)
    sm = to_dev(np.array([pool.slot(pos)], np.int32))
    cl = to_dev(np.array([pos + 1], np.int32))
    rc = ssdq.decode_layer(store, layer, cfg, hd, pos, pool.dev[0], pool.dev[1], pool.dev[2], pool.dev[3], BLOCK,
                           bt, pool.max_blocks, sm, cl, pool.max_blocks * BLOCK, scratch=scratch)
    assert rc == 0, ssdq.last_error()
    out = from_dev(hd)
    raw = from_dev(scratch)
    got = {name: raw[off:off + 4 * n].view(np.float32).copy() for name, (off, n) in
           ((k, (offs[k], steps[k])) for k in steps)}
    return out, got


def step_sizes(L):
    q_dim, kv_dim = L.n_head * L.hd, L.n_kv * L.hd
    return {"attn_in": L.n_embd, "q": q_dim, "k": kv_dim, "v": kv_dim, "attn": q_dim, "attn_out": L.n_embd,
            "ffn_in": L.n_embd, "ffn_h": L.n_ff, "ffn_out": L.n_embd}


def check_steps(L, hidden, pos, pool, before, after, got, out, theta, what):
    """Every step against the oracle on the device's own input to that step;
    before / after: the device pool's (k codes, k scales, v codes, v scales)
    around the call."""
    n_embd, q_dim, kv_dim = L.n_embd, L.n_head * L.hd, L.n_kv * L.hd
    if L.has("attn_norm"):
        assert_close(got["attn_in"], o.rmsnorm(hidden, L.norm("attn_norm"), EPS), f"{what}: attention norm")
    else:
        assert bits_equal(got["attn_in"], hidden), f"{what}: attention input copy"
    x = got["attn_in"]
    for name, t, rows in (("q", "attn_q", q_dim), ("k", "attn_k", kv_dim)):
        ex = o.matvec_exact(L.dt(t), L.w(t), x, rows, n_embd)
        assert_propagated(got[name], rope_double(ex, L.hd, pos, theta), rope_bound(ex, L.hd, pos, theta),
                          f"{what}: {name} + RoPE")
    rv, _ = o.matvec(L.dt("attn_v"), L.w("attn_v"), x, kv_dim, n_embd, threads=16)
    assert_close_attributed(got["v"], rv, o.matvec_exact(L.dt("attn_v"), L.w("attn_v"), x, kv_dim, n_embd),
                            f"{what}: v")
    # the pool: this token's row is the INT8 quantization of the device's k / v
    # (bit-exact), every other row unchanged
    r = pool.slot(pos)
    kc, ks = o.quantize_rows(got["k"], 1, kv_dim)
    vc, vs = o.quantize_rows(got["v"], 1, kv_dim)
    kca, ksa, vca, vsa = after
    assert bits_equal(kca[r * kv_dim:(r + 1) * kv_dim], kc) and bits_equal(ksa[r:r + 1], ks), f"{what}: K row"
    assert bits_equal(vca[r * kv_dim:(r + 1) * kv_dim], vc) and bits_equal(vsa[r:r + 1], vs), f"{what}: V row"
    keep = np.ones(len(ksa), bool)
    keep[r] = False
    kk = np.repeat(keep, kv_dim)
    for a, b in zip(after, before):
        m = kk if a.size == kk.size else keep
        assert bits_equal(a[m], b[m]), f"{what}: a pool row other than the token's changed"
    att = o.paged_attention_int8(got["q"], kca, ksa, vca, vsa, pool.table, np.array([pos + 1]), 1,
                                 L.n_head, L.n_kv, L.hd, BLOCK, pool.max_blocks, threads=16)
    assert_close(got["attn"], att, f"{what}: paged attention")
    wo = L.w("attn_output")
    ro, _ = o.matvec(L.dt("attn_output"), wo, got["attn"], n_embd, q_dim, threads=16)
    assert_close_attributed(got["attn_out"], ro, o.matvec_exact(L.dt("attn_output"), wo, got["attn"], n_embd,
                                                                q_dim), f"{what}: output projection")
    h_mid = (hidden + got["attn_out"]).astype(np.float32)  # the residual add, fp32
    if L.has("ffn_norm"):
        _, fin = o.fused_post_attn_norm(hidden, got["attn_out"], L.norm("ffn_norm"), EPS)
        assert_close(got["ffn_in"], fin, f"{what}: post-attention norm")
        fin_dev = got["ffn_in"]
    else:
        fin_dev = h_mid
    if not L.has("ffn_gate", "ffn_up", "ffn_down"):
        assert bits_equal(out, h_mid), f"{what}: attention residual"
        return
    g = o.matvec_exact(L.dt("ffn_gate"), L.w("ffn_gate"), fin_dev, L.n_ff, n_embd)
    u = o.matvec_exact(L.dt("ffn_up"), L.w("ffn_up"), fin_dev, L.n_ff, n_embd)
    ex, extra = swiglu_propagated(g, u)
    assert_propagated(got["ffn_h"], ex, extra, f"{what}: SwiGLU")
    wd = L.w("ffn_down")
    rd, _ = o.matvec(L.dt("ffn_down"), wd, got["ffn_h"], n_embd, L.n_ff, threads=16)
    assert_close_attributed(got["ffn_out"], rd, o.matvec_exact(L.dt("ffn_down"), wd, got["ffn_h"], n_embd, L.n_ff),
                            f"{what}: down projection")
    assert bits_equal(out, (h_mid + got["ffn_out"]).astype(np.float32)), f"{what}: FFN residual"


LLAMA = dict(n_embd=4096, n_head=32, n_kv=8, hd=128, n_ff=14336)
Q4KM = {"attn_q": Q4_K, "attn_k": Q4_K, "attn_v": Q4_K, "attn_output": Q4_K, "ffn_gate": Q4_K, "ffn_up": Q4_K,
        "ffn_down": Q6_K}
MIXED = dict(Q4KM, attn_v=Q6_K, ffn_up=Q8_0)
SMALL = dict(n_embd=1024, n_head=8, n_kv=2, hd=128, n_ff=2816)
CASES = [
    # (id, shape, types, norm type, dropped tensors, earlier tokens, theta, hidden scale)
    ("llama3_8b_q4k", LLAMA, Q4KM, F32, (), 300, 500000.0, 1.0),          # fused QKV + RoPE and SwiGLU kernels
    ("llama3_8b_mixed_f16norm", LLAMA, MIXED, F16, (), 77, 500000.0, 1.0),  # separate launches; F16 norms
    ("small_no_ffn_norm", SMALL, Q4KM, F32, ("ffn_norm",), 40, 10000.0, 1.0),
    ("small_no_ffn", SMALL, Q4KM, F32, ("ffn_down",), 5, 10000.0, 1.0),
    # without the norm the hidden state feeds the projections as it is
    ("small_no_attn_norm_hd64", dict(SMALL, n_head=16, n_kv=4, hd=64, n_ff=2048), Q4KM, F32, ("attn_norm",), 33,
     10000.0, 1.0),
    # the norm-fused kernels with Q8_0 q/k/v (2688 row pairs: 10 or 11 per CU
    # on 256 CUs) and Q4_0 gate/up, a 3840-wide attention output
    ("q8_0_qkv_30_heads_q4_0_ffn", dict(LLAMA, n_head=30, n_kv=6, n_ff=11008),
     dict(Q4KM, attn_q=Q8_0, attn_k=Q8_0, attn_v=Q8_0, ffn_gate=Q4_0, ffn_up=Q4_0), F32, (), 130, 500000.0, 1.0),
]


@pytest.mark.parametrize("cid,shape,types,norm_type,drop,ctx,theta,hscale", CASES, ids=[c[0] for c in CASES])
def test_decode_layer_from_resident_weights(cid, shape, types, norm_type, drop, ctx, theta, hscale):
    layer = 3
    L = Layer(shape["n_embd"], shape["n_head"], shape["n_kv"], shape["hd"], shape["n_ff"], types, 4100, norm_type,
              drop)
    kv_dim = L.n_kv * L.hd
    cfg = ssdq.layer_config(L.n_embd, L.n_head, L.n_kv, L.hd, L.n_ff, theta, EPS)
    nbytes, offs = ssdq.decode_layer_scratch(cfg)
    scratch = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    g = synth.rng(4200)
    hidden0 = (g.standard_normal(L.n_embd) * hscale).astype(np.float32)
    hidden1 = (g.standard_normal(L.n_embd) * hscale).astype(np.float32)

    # the oracle composition first: its k / v rms sets the earlier tokens' scale
    probe = Pool(kv_dim, 0, 64, 96, (1.0, 1.0), 4300)
    _, st = oracle_layer(L, hidden0, ctx, probe, theta)
    kv_rms = (float(np.sqrt(np.mean(st["k"] ** 2))), float(np.sqrt(np.mean(st["v"] ** 2)))) if "k" in st else \
        (1.0, 1.0)
    pool = Pool(kv_dim, ctx, 64, 96, kv_rms, 4301).upload()
    ref_pool = Pool(kv_dim, ctx, 64, 96, kv_rms, 4301)

    announce("decode layer", cid, "upload")
    store = ssdq.WeightStore()
    try:
        up = L.upload(store, layer)
        assert len(store) == len(L.t) and store.nbytes == up
        assert store.find(f"blk.{layer}.attn_q.weight")[1:3] == (L.dt("attn_q"), L.t["attn_q"][1])
        assert store.find(f"blk.{layer + 1}.attn_q.weight") is None
        steps = step_sizes(L)
        for tok, (hid, pos) in enumerate(((hidden0, ctx), (hidden1, ctx + 1))):
            announce("decode layer", cid, "token", tok, "position", pos)
            before = pool.from_device()
            out, got = run_gpu_layer(store, layer, cfg, hid, pos, pool, scratch, offs, steps)
            assert np.all(np.isfinite(out))
            check_steps(L, hid, pos, pool, before, pool.from_device(), got, out, theta, f"{cid} token {tok}")
            # end to end: the oracle composition from the same hidden state, its
            # own pool (the earlier tokens, then its own appends)
            ref, st = oracle_layer(L, hid, pos, ref_pool, theta)
            scale = term_scale(L, hid, st)
            err = np.abs(out.astype(np.float64) - ref)
            bound = ATOL + E2E_RTOL * scale
            print(f"{cid} token {tok}: layer output max |gpu - ref| / term scale = {np.max(err / scale):.2e}")
            assert np.all(err <= bound), (f"{cid} token {tok}: layer output: {int((err > bound).sum())} outside; "
                                          f"worst {int(np.argmax(err / bound))}")
            if "attn" in st:
                spread = effective_positions(L, st["q"], ref_pool, pos)
                print(f"{cid} token {tok}: attention over {pos + 1} positions, effective {spread:.1f}")
                assert spread > 1.5 or pos < 8, "one-hot attention: the case would not test the weighting"
    finally:
        store.close()
        torch.cuda.synchronize()


def test_decode_layer_hidden_near_fp32_max():
    """Hidden values near FLT_MAX.  The norms' fp32 sums of squares overflow, so
    the reference's inv_rms is 0 and its normalised vectors are 0: q, k, v and
    the FFN are zero, and the layer output is hidden + the attention output.
    The norm-fused kernels stage h * w and scale the dot products by inv_rms;
    here some of those products overflow fp32 (|h| 3e38, w > 1.2), which they
    stage scaled by a power of two, so the outputs are those zeros, not NaN."""
    shape = dict(n_embd=4096, n_head=8, n_kv=2, hd=128, n_ff=2048)  # fused: 768 and 2048 row pairs
    L = Layer(shape["n_embd"], shape["n_head"], shape["n_kv"], shape["hd"], shape["n_ff"], Q4KM, 4500)
    kv_dim, theta, pos, layer = L.n_kv * L.hd, 500000.0, 40, 2
    cfg = ssdq.layer_config(L.n_embd, L.n_head, L.n_kv, L.hd, L.n_ff, theta, EPS)
    nbytes, offs = ssdq.decode_layer_scratch(cfg)
    scratch = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    hidden = synth.rng(4501).standard_normal(L.n_embd).astype(np.float32)
    big = np.flatnonzero((L.norm("attn_norm") > 1.2) & (L.norm("ffn_norm") > 1.2))[:8]
    assert big.size == 8
    hidden[big] = np.where(np.arange(8) % 2, 3.0e38, -3.0e38).astype(np.float32)
    pool = Pool(kv_dim, pos, 8, 16, (1.0, 1.0), 4502).upload()
    ref_pool = Pool(kv_dim, pos, 8, 16, (1.0, 1.0), 4502)
    store = ssdq.WeightStore()
    try:
        L.upload(store, layer)
        announce("decode layer near FLT_MAX", "position", pos)
        before = pool.from_device()
        out, got = run_gpu_layer(store, layer, cfg, hidden, pos, pool, scratch, offs, step_sizes(L))
        assert np.all(np.isfinite(out))
        for name in ("attn_in", "q", "k", "v", "ffn_in", "ffn_h", "ffn_out"):
            assert not np.any(got[name]), f"{name}: not all zero"
        check_steps(L, hidden, pos, pool, before, pool.from_device(), got, out, theta, "near FLT_MAX")
        ref, st = oracle_layer(L, hidden, pos, ref_pool, theta)
        assert not np.any(st["q"]) and not np.any(st["ffn_h"])
        err = np.abs(out.astype(np.float64) - ref)
        assert np.all(err <= ATOL + E2E_RTOL * term_scale(L, hidden, st))
    finally:
        store.close()
        torch.cuda.synchronize()


def abs_matvec(dtype, w, x, out_dim, in_dim):
    """|W| |x| over the dequantized elements (bit-exact values)"""
    e, rc = o.matvec_elements(dtype, w, out_dim, in_dim)
    assert rc == 0
    return np.abs(e.astype(np.float64)) @ np.abs(np.asarray(x, np.float64))


def term_scale(L, hidden, st):
    """|hidden| + |Wo| |a| + |W_down| |h|: the magnitude of the terms summed
    into each layer output (the oracle's a and h)"""
    s = np.abs(hidden.astype(np.float64))
    if "attn" in st:
        s = s + abs_matvec(L.dt("attn_output"), L.w("attn_output"), st["attn"], L.n_embd, L.n_head * L.hd)
    if "ffn_h" in st:
        s = s + abs_matvec(L.dt("ffn_down"), L.w("ffn_down"), st["ffn_h"], L.n_embd, L.n_ff)
    return s


def effective_positions(L, q, pool, pos):
    """exp(entropy) of each head's softmax over the pool's dequantized keys,
    averaged over heads: the case is neither one-hot nor uniform."""
    kv_dim = L.n_kv * L.hd
    rows = [pool.slot(p) for p in range(pos + 1)]
    k = np.stack([pool.kc[r * kv_dim:(r + 1) * kv_dim].astype(np.float64) * pool.ks[r] for r in rows])
    out = []
    for h in range(L.n_head):
        kvh = h // (L.n_head // L.n_kv)
        s = k[:, kvh * L.hd:(kvh + 1) * L.hd] @ q[h * L.hd:(h + 1) * L.hd].astype(np.float64) / np.sqrt(L.hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out.append(np.exp(-(p * np.log(np.maximum(p, 1e-300))).sum()))
    return float(np.mean(out))


def test_decode_layer_skips_without_attention_tensors():
    """Without all four attention tensors the reference leaves the hidden
    state as it is (transformer.rs:326-331)."""
    L = Layer(1024, 8, 2, 128, 2816, Q4KM, 4400, drop=("attn_v",))
    cfg = ssdq.layer_config(1024, 8, 2, 128, 2816, 10000.0, EPS)
    pool = Pool(256, 3, 8, 8, (1.0, 1.0), 4401).upload()
    nbytes, offs = ssdq.decode_layer_scratch(cfg)
    scratch = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    hidden = synth.rng(4402).standard_normal(1024).astype(np.float32)
    store = ssdq.WeightStore()
    try:
        L.upload(store, 0)
        announce("decode layer without attn_v")
        out, got = run_gpu_layer(store, 0, cfg, hidden, 3, pool, scratch, offs, {"attn_in": 1024})
        assert bits_equal(out, hidden)
        assert_close(got["attn_in"], o.rmsnorm(hidden, L.norm("attn_norm"), EPS), "attention norm")
        after = pool.from_device()
        assert bits_equal(after[1], pool.ks) and bits_equal(after[0], pool.kc)  # nothing appended
    finally:
        store.close()


def test_decode_layer_rejects_mismatched_shapes_before_launch():
    L = Layer(1024, 8, 2, 128, 2816, Q4KM, 4500)
    store = ssdq.WeightStore()
    try:
        L.upload(store, 0)
        with pytest.raises(ssdq.SsdqError) as e:  # a layer with 4 KV heads expects wider attn_k
            dummy = torch.zeros(1024, dtype=torch.float32, device="cuda")
            ssdq.decode_layer(store, 0, ssdq.layer_config(1024, 8, 4, 128, 2816, 1e4), dummy, 0, dummy, dummy,
                              dummy, dummy, BLOCK, dummy, 1, dummy, dummy, 16)
        assert "attn_k" in str(e.value)
        with pytest.raises(ssdq.SsdqError):  # duplicate name
            store.put("blk.0.attn_q.weight", Q4_K, (1024, 1024), L.w("attn_q"))
        with pytest.raises(ssdq.SsdqError):  # bytes disagree with dims and type
            store.put("blk.9.x.weight", Q4_K, (1024, 8), L.w("attn_q")[:100])
    finally:
        store.close()


def test_decode_layer_graph_replay_matches_eager():
    """The layer captured into a HIP graph (after an eager call on the capture
    stream sizes its workspaces) and replayed, with eager work between the
    replays: every replay leaves the hidden state and the pool bit-identical
    to an eager call on the same inputs."""
    L = Layer(1024, 8, 2, 128, 2816, Q4KM, 4600)
    cfg = ssdq.layer_config(1024, 8, 2, 128, 2816, 10000.0, EPS)
    pool = Pool(256, 50, 8, 8, (1.0, 1.0), 4601).upload()
    hidden0 = synth.rng(4602).standard_normal(1024).astype(np.float32)
    pos = 50
    store = ssdq.WeightStore()
    side = torch.cuda.Stream()
    try:
        L.upload(store, 0)
        h = to_dev(hidden0)
        h_in = to_dev(hidden0)
        bt = to_dev(pool.table)
        sm = to_dev(np.array([pool.slot(pos)], np.int32))
        cl = to_dev(np.array([pos + 1], np.int32))
        kc, ks, vc, vs = pool.dev

        def call():
            return ssdq.decode_layer(store, 0, cfg, h, pos, kc, ks, vc, vs, BLOCK, bt, pool.max_blocks, sm, cl,
                                     pool.max_blocks * BLOCK, stream=side)

        announce("decode layer: eager reference on the capture stream")
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            assert call() == 0
        side.synchronize()
        ref_h = from_dev(h)
        ref_pool = pool.from_device()
        g = torch.cuda.CUDAGraph()
        h.copy_(h_in)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=side):
            assert call() == 0
        torch.cuda.synchronize()
        for rep in range(3):
            announce("decode layer: graph replay", rep)
            h.copy_(h_in)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert bits_equal(from_dev(h), ref_h), f"replay {rep}: hidden state"
            for a, b in zip(pool.from_device(), ref_pool):
                assert bits_equal(a, b), f"replay {rep}: pool"
            # unrelated eager work on the capture stream between replays
            with torch.cuda.stream(side):
                ssdq.rmsnorm(h_in, None, h_in, 1e-5, None, torch.empty_like(h_in), 1024, stream=side)
            side.synchronize()
        del g
        torch.cuda.synchronize()
    finally:
        store.close()


def test_two_decoder_layers_chained():
    """Layers 0 and 1 (different weights, one pool each) applied in turn to one
    token, against the oracle's composition chained the same way; each layer's
    output held to the end-to-end bar against the oracle run from the device's
    own input to that layer."""
    shape = dict(n_embd=2048, n_head=16, n_kv=4, hd=128, n_ff=5632)
    layers = [Layer(shape["n_embd"], shape["n_head"], shape["n_kv"], shape["hd"], shape["n_ff"], Q4KM, 4700 + 100 * i)
              for i in range(2)]
    cfg = ssdq.layer_config(2048, 16, 4, 128, 5632, 500000.0, EPS)
    nbytes, offs = ssdq.decode_layer_scratch(cfg)
    scratch = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    ctx = 123
    pools = [Pool(512, ctx, 16, 24, (1.0, 1.0), 4800 + i).upload() for i in range(2)]
    ref_pools = [Pool(512, ctx, 16, 24, (1.0, 1.0), 4800 + i) for i in range(2)]
    hid = synth.rng(4900).standard_normal(2048).astype(np.float32)
    store = ssdq.WeightStore()
    try:
        for i, L in enumerate(layers):
            L.upload(store, i)
        assert len(store) == 18
        steps = step_sizes(layers[0])
        h_dev_in = hid
        for i, L in enumerate(layers):
            announce("two layers: layer", i)
            out, got = run_gpu_layer(store, i, cfg, h_dev_in, ctx, pools[i], scratch, offs, steps)
            ref, st = oracle_layer(L, h_dev_in, ctx, ref_pools[i], 500000.0)
            scale = term_scale(L, h_dev_in, st)
            err = np.abs(out.astype(np.float64) - ref)
            assert np.all(err <= ATOL + E2E_RTOL * scale), f"layer {i}: {int((err > ATOL + E2E_RTOL * scale).sum())}"
            print(f"layer {i}: max |gpu - ref| / term scale = {np.max(err / scale):.2e}")
            h_dev_in = out
    finally:
        store.close()
