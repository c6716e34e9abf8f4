"""Batch-1 / small-batch matvec parity on activations with massive channels.

Real decoder hidden states carry a few channels 10^3-10^4 times larger than
the rest, in many 32-element groups.  The matvec kernels carry x per
32-element group as an integer of at most 2^30 against the group's largest
magnitude, so an element 2^k below its group's maximum keeps 30 - k bits
(with 22 bits, 3-9 of these 14336 outputs per case fell outside the
tolerance).
These cases check that the outputs still meet the stated tolerance against
the reference's serial fp32 chain (matvec_*_cpu, src/metal/compute.rs:680-925),
with the exact-sum substitution only where that chain is itself off, at the
Llama-3-8B FFN shape 14336 x 4096 for Q4_K, Q4_0 and Q8_0, batch 1 and 8.
"""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, assert_close_attributed, empty_dev, from_dev, to_dev
from ssdq import synth

pytestmark = pytest.mark.gpu


def massive_activations(batch, in_dim, seed, frac=0.01, lo=1e3, hi=1e4):
    """N(0,1) rows with ~frac of the channels at +-U[lo, hi] (the same channels
    in every row, as in real hidden states), spread over many 32-element groups."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((batch, in_dim)).astype(np.float32)
    n = max(1, int(round(frac * in_dim)))
    ch = g.choice(in_dim, n, replace=False)
    mag = g.uniform(lo, hi, (batch, n)) * g.choice([-1.0, 1.0], (batch, n))
    x[:, ch] = mag.astype(np.float32)
    return x, ch


@pytest.mark.parametrize("dtype", [ssdq.Q4_K, ssdq.Q4_0, ssdq.Q8_0])
@pytest.mark.parametrize("batch", [1, 8])
def test_massive_activation_channels(dtype, batch):
    out_dim, in_dim = 14336, 4096
    w = synth.quant_weights(dtype, out_dim, in_dim, 1300 + dtype)
    x, ch = massive_activations(batch, in_dim, 1400 + batch)
    groups = np.unique(ch // 32).size
    assert groups >= 30  # the outliers sit in many different groups
    announce("matvec massive activations", ssdq.TYPE_NAMES[dtype], out_dim, in_dim, batch, groups)
    y = empty_dev(out_dim * batch, torch.float32)
    assert ssdq.matvec(dtype, to_dev(w), to_dev(x), y, out_dim, in_dim, batch) == 0
    got = from_dev(y).reshape(batch, out_dim)
    # every output of the first and last activation row; rows between on a sample
    rows = np.arange(out_dim)
    for b in range(batch):
        sel = rows if b in (0, batch - 1) else rows[::7]
        rb = w.size // out_dim
        wsel = w.reshape(out_dim, rb)[sel].ravel()
        ref, _ = o.matvec(dtype, wsel, x[b], sel.size, in_dim, threads=16)
        ex = o.matvec_exact(dtype, wsel, x[b], sel.size, in_dim)
        assert_close_attributed(got[b, sel], ref, ex, f"{ssdq.TYPE_NAMES[dtype]} massive b{b}/{batch}")
