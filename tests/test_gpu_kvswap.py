"""Paged INT8 KV swap slots through the C ABI: swap-out packs pool blocks into
the reference's SwapQuantMode::Int8 slot bytes (SwapFile::write_block,
src/ssd/block_swap.rs:187-252), bit for bit, into device memory or mapped
pinned host memory; swap-in restores codes, scales and num_filled exactly, and
the restored block dequantizes to what SwapFile::read_block returns
(block_swap.rs:283-370)."""
import numpy as np
import pytest
import torch

import ssdq
import ssdq_oracle as o
from helpers import announce, from_dev, to_dev

pytestmark = pytest.mark.gpu


def pool(n_blocks, bs, kv, seed):
    g = np.random.default_rng(seed)
    kf = g.standard_normal((n_blocks * bs, kv), dtype=np.float32)
    vf = g.standard_normal((n_blocks * bs, kv), dtype=np.float32)
    kf[5] = 0.0  # an all-zero row: scale 0, codes 0
    kc, ks, vc, vs = (torch.empty(n_blocks * bs * kv, dtype=torch.int8, device="cuda"),
                      torch.empty(n_blocks * bs, device="cuda"),
                      torch.empty(n_blocks * bs * kv, dtype=torch.int8, device="cuda"),
                      torch.empty(n_blocks * bs, device="cuda"))
    ssdq.kv_quantize_rows(to_dev(kf), kc, ks, n_blocks * bs, kv)
    ssdq.kv_quantize_rows(to_dev(vf), vc, vs, n_blocks * bs, kv)
    return kf, vf, (kc, ks, vc, vs)


@pytest.mark.parametrize("bs,kv,host", [(16, 1024, False), (16, 1024, True), (4, 8, False), (1, 128, True),
                                        (32, 256, False)])
def test_swap_out_matches_reference_slots_and_round_trips(bs, kv, host):
    n_pool = 40
    kf, vf, (kc, ks, vc, vs) = pool(n_pool, bs, kv, bs * kv)
    g = np.random.default_rng(kv)
    ids = g.permutation(n_pool)[:17].astype(np.int32)
    nfill = g.integers(0, bs + 1, ids.size).astype(np.uint32)
    sb = ssdq.kv_slot_bytes(bs, kv)
    assert sb == o.kv_slot_bytes(bs, kv)
    if host:
        slots = torch.zeros(ids.size * sb, dtype=torch.uint8).pin_memory()
    else:
        slots = torch.zeros(ids.size * sb, dtype=torch.uint8, device="cuda")
    announce("kv swap out", bs, kv, "pinned host" if host else "device")
    ssdq.kv_swap_out(kc, ks, vc, vs, to_dev(ids), to_dev(nfill), ids.size, bs, kv, n_pool, slots)
    torch.cuda.synchronize()
    got = slots.cpu().numpy().reshape(ids.size, sb)
    for j, b in enumerate(ids):
        want = o.kv_swap_write(kf[b * bs:(b + 1) * bs], vf[b * bs:(b + 1) * bs], bs, kv, int(nfill[j]))
        assert np.array_equal(got[j], want), f"slot {j} (block {b})"
    # swap in to other physical blocks of a cleared pool
    dst = np.roll(ids, 3).astype(np.int32)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    ks2, vs2 = torch.zeros_like(ks), torch.zeros_like(vs)
    nf_out = torch.zeros(ids.size, dtype=torch.int32, device="cuda")
    announce("kv swap in", bs, kv)
    ssdq.kv_swap_in(slots, to_dev(dst), ids.size, bs, kv, n_pool, kc2, ks2, vc2, vs2, nf_out)
    kcn, ksn, vcn, vsn = (from_dev(t) for t in (kc, ks, vc, vs))
    kc2n, ks2n, vc2n, vs2n = (from_dev(t) for t in (kc2, ks2, vc2, vs2))
    for j, (b, d) in enumerate(zip(ids, dst)):
        r0, r1, d0, d1 = b * bs, (b + 1) * bs, d * bs, (d + 1) * bs
        assert np.array_equal(kc2n[d0 * kv:d1 * kv], kcn[r0 * kv:r1 * kv])
        assert np.array_equal(vc2n[d0 * kv:d1 * kv], vcn[r0 * kv:r1 * kv])
        assert np.array_equal(ks2n[d0:d1].view(np.uint32), ksn[r0:r1].view(np.uint32))
        assert np.array_equal(vs2n[d0:d1].view(np.uint32), vsn[r0:r1].view(np.uint32))
        # and the restored block dequantizes to read_block's f32 rows
        kr, vr, nf = o.kv_swap_read(got[j], bs, kv)
        kd = torch.empty(bs * kv, device="cuda")
        ssdq.kv_dequantize_rows(kc2[d0 * kv:d1 * kv], ks2[d0:d1], kd, bs, kv)
        assert np.array_equal(from_dev(kd).view(np.uint32), kr.view(np.uint32))
        assert nf == nfill[j]
    assert np.array_equal(from_dev(nf_out).astype(np.uint32), nfill)
    untouched = np.setdiff1d(np.arange(n_pool), dst)
    for d in untouched[:5]:
        assert not kc2n[d * bs * kv:(d + 1) * bs * kv].any()


def test_invalid_ids_give_zero_slots_and_are_skipped():
    bs, kv, n_pool = 4, 64, 6
    _, _, (kc, ks, vc, vs) = pool(n_pool, bs, kv, 3)
    ids = np.array([2, -1, 6, 1000], np.int32)
    sb = ssdq.kv_slot_bytes(bs, kv)
    slots = torch.full((ids.size * sb,), 0x5A, dtype=torch.uint8, device="cuda")
    announce("kv swap invalid ids")
    ssdq.kv_swap_out(kc, ks, vc, vs, to_dev(ids), None, ids.size, bs, kv, n_pool, slots)
    got = from_dev(slots).reshape(ids.size, sb)
    assert got[0].any() and not got[1:].any()
    assert not got[0][-4:].any()  # num_filled NULL -> 0
    before = from_dev(kc).copy()
    ssdq.kv_swap_in(slots, to_dev(np.array([-5, 7, 99, 1], np.int32)), 4, bs, kv, n_pool, kc, ks, vc, vs, None)
    after = from_dev(kc)
    assert not after[1 * bs * kv:2 * bs * kv].any()  # slot 3 (zeros) restored into block 1
    mask = np.ones(after.size, bool)
    mask[1 * bs * kv:2 * bs * kv] = False
    assert np.array_equal(after[mask], before[mask])


def test_swap_rejects_bad_arguments():
    z = torch.zeros(1024, dtype=torch.int8, device="cuda")
    f = torch.zeros(64, device="cuda")
    ids = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(ssdq.SsdqError):  # kv_dim not a multiple of 4
        ssdq.kv_swap_out(z, f, z, f, ids, None, 1, 2, 6, 1, z)
    with pytest.raises(ssdq.SsdqError):  # misaligned slots
        ssdq.kv_swap_out(z, f, z, f, ids, None, 1, 2, 8, 1, z[1:])
