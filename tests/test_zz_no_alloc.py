"""The allocation-free paged INT8 decode attention
(ssdq_paged_attention_int8_noalloc_dev) against the allocating entry point
(ssdq_paged_attention_int8_dev): same kernels, same split plan, so the outputs
must be bit-identical.  Two calls in a row on the shared static scratch, the
second with a smaller input (fewer sequences, shorter context), each compared
with the allocating entry point on the same input; a call whose partials
exceed the static maximum is rejected.  The oracle check of the kernels
themselves is tests/test_gpu_attention.py."""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, from_dev, to_dev
from ssdq import synth

pytestmark = pytest.mark.gpu


def _case(n_seq, n_head, n_kv, hd, bs, ctx, seed):
    mb = (ctx + bs - 1) // bs
    g = np.random.default_rng(seed)
    tables = synth.block_tables(n_seq, mb, seed + 1)
    rows = n_seq * mb * bs
    kf = g.standard_normal((rows, n_kv * hd)).astype(np.float32)
    vf = g.standard_normal((rows, n_kv * hd)).astype(np.float32)
    kc, ks = o.quantize_rows(kf, rows, n_kv * hd)
    vc, vs = o.quantize_rows(vf, rows, n_kv * hd)
    q = g.standard_normal((n_seq, n_head, hd)).astype(np.float32)
    lens = np.array([ctx - (7 * i) % max(ctx // 3, 1) for i in range(n_seq)], np.int32)
    lens[0] = ctx
    d = [to_dev(a) for a in (q, kc, ks, vc, vs, tables, lens)]
    return d, (n_seq, n_head, n_kv, hd, bs, mb, int(lens.max())), (q, kc, ks, vc, vs, tables, lens)


def _run(fn, d, dims):
    n_seq, n_head, n_kv, hd, bs, mb, max_ctx = dims
    out = torch.full((n_seq * n_head * hd,), float("nan"), device="cuda")
    fn(*d, out, n_seq, n_head, n_kv, hd, bs, mb, max_ctx)
    return from_dev(out)


def test_noalloc_matches_allocating_entry_point():
    # first call: config-5 heads at 8k context; second: smaller (3 sequences, 700 tokens)
    for label, args in (("large", (8, 32, 8, 128, 16, 8192, 11)), ("small", (3, 32, 8, 128, 16, 700, 12))):
        d, dims, host = _case(*args)
        announce("noalloc attention", label, args)
        got = _run(ssdq.paged_attention_int8_noalloc, d, dims)
        want = _run(ssdq.paged_attention_int8, d, dims)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), label
        if label == "small":  # and the oracle, on the small case
            q, kc, ks, vc, vs, tables, lens = host
            n_seq, n_head, n_kv, hd, bs, mb, _ = dims
            ref = o.paged_attention_int8(q, kc, ks, vc, vs, tables, lens, n_seq, n_head, n_kv, hd, bs, mb,
                                         threads=8)
            err = np.abs(got - ref) - (1e-4 + 1e-3 * np.abs(ref))
            assert err.max() <= 0


def test_noalloc_rejects_oversized_partials():
    # 4096 sequences x 64 heads need at least 4096 * 64 * (128 + 2) * 4 bytes of
    # partials (136 MB, one split) against the 16 MiB scratch: the entry point
    # rejects the call before any launch, so the small buffers are never read
    t = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    ctx = torch.full((4096,), 1024, dtype=torch.int32, device="cuda")
    announce("noalloc attention: oversized request")
    with pytest.raises(ssdq.SsdqError) as ei:
        ssdq.paged_attention_int8_noalloc(t, t, t, t, t, t, ctx, t, 4096, 64, 8, 128, 16, 64, 1024)
    assert "scratch" in str(ei.value)
