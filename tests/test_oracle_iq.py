"""Pins the oracle's IQ2_XXS / IQ2_XS / IQ3_XXS / IQ3_S matvecs
(src/metal/compute.rs:1983-2238) and the lattice code books they read
(ssd-llm_amd/csrc/iq_grids.h):
  * the tables hash to tests/golden/iq_grids.json (written from the reference's
    tables by tests/golden/make_iq_grids.py) and hold the entries the
    reference's own tests assert (compute.rs:2847-2958);
  * the sign table is the parity closed form, checked against entries of the
    reference's KSIGNS_IQ2XS (compute.rs:1964-1973);
  * the reference's known-answer tests for the four types;
  * independent encoders place grid indices, sign indices / masks, high index
    bits and scales; the matvec on unit vectors and the element decoder return
    exactly the values the fields define;
  * the matvec equals the serial fp32 sum in the reference's order (IQ3
    alternates j and j+4 inside each group of 8) and stays within the
    serial-sum bound of the exact sum."""
import hashlib
import json
import os
import re

import numpy as np
import pytest

import encoders as enc
import ssdq_oracle as o

IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S = 16, 17, 18, 21
HERE = os.path.dirname(os.path.abspath(__file__))
HDR = os.path.join(HERE, "..", "ssd-llm_amd", "csrc", "iq_grids.h")


def grids():
    src = open(HDR).read()
    out = {}
    for name, ty in (("iq2xxs", 8), ("iq2xs", 8), ("iq3xxs", 4), ("iq3s", 4)):
        body = re.search(r"#define SSDQ_%s_GRID_INIT \{(.*?)\n\}" % name.upper(), src, re.S).group(1)
        out[name] = [int(v, 16) for v in re.findall(r"0x[0-9a-f]+", body)], ty
    return out


G = grids()


def gbytes(name, idx):
    v, n = G[name]
    return [(v[idx] >> (8 * j)) & 0xFF for j in range(n)]


def ksigns(i):
    return i | ((bin(i).count("1") & 1) << 7)


def test_tables_match_the_reference():
    meta = json.load(open(os.path.join(HERE, "golden", "iq_grids.json")))
    for name, key in (("iq2xxs", "IQ2XXS_GRID"), ("iq2xs", "IQ2XS_GRID"), ("iq3xxs", "IQ3XXS_GRID"),
                      ("iq3s", "IQ3S_GRID")):
        v, n = G[name]
        raw = b"".join(x.to_bytes(n, "little") for x in v)
        assert len(v) == meta[key]["entries"] and hashlib.sha256(raw).hexdigest() == meta[key]["sha256"]
    # compute.rs:2847-2958
    assert G["iq3xxs"][0][0] == 0x04040404 and G["iq3xxs"][0][255] == 0x3E341C04
    assert G["iq3s"][0][0] == 0x01010101 and G["iq3s"][0][511] == 0x0F0F0101
    assert G["iq2xxs"][0][0] == 0x0808080808080808 and G["iq2xxs"][0][255] == 0x2B2B2B1908081908
    assert G["iq2xs"][0][0] == 0x0808080808080808 and G["iq2xs"][0][511] == 0x2B2B2B2B2B2B2B2B
    # the reference's KSIGNS_IQ2XS, first and last entries
    assert [ksigns(i) for i in range(10)] == [0, 129, 130, 3, 132, 5, 6, 135, 136, 9]
    assert [ksigns(i) for i in range(123, 128)] == [123, 252, 125, 126, 255]


def _f16b(v):
    b = int(enc.f16_bits(v))
    return b & 0xFF, b >> 8


def _y(dtype, blk, x):
    y, rc = o.matvec(dtype, np.asarray(blk, np.uint8), np.asarray(x, np.float32), 1, 256)
    assert rc == 0
    return y[0]


def test_reference_known_answers():
    ones = np.ones(256, np.float32)
    b = np.zeros(98, np.uint8)  # compute.rs:2747-2789
    b[0], b[1] = _f16b(1.0)
    assert abs(_y(IQ3_XXS, b, ones) - 256.0) < 1.0
    b[66:70] = np.array([127, 0, 0, 0], np.uint8)
    assert abs(_y(IQ3_XXS, b, ones) - 240.0) < 1.0
    b = np.zeros(110, np.uint8)  # compute.rs:2791-2845
    b[0], b[1] = _f16b(1.0)
    assert abs(_y(IQ3_S, b, ones) - 256.0) < 1.0
    b[74] = 0xFF
    assert abs(_y(IQ3_S, b, ones) - 240.0) < 1.0
    b = np.zeros(110, np.uint8)
    b[0], b[1] = _f16b(0.5)
    b[106:110] = 0x31
    assert abs(_y(IQ3_S, b, ones) - 640.0) < 2.0
    b = np.zeros(66, np.uint8)  # compute.rs:2865-2908
    b[1] = 0x3C
    assert abs(_y(IQ2_XXS, b, ones) - 256.0) < 1.0
    b[6] = 0x7F
    assert abs(_y(IQ2_XXS, b, ones)) > 0.0
    b = np.zeros(74, np.uint8)  # compute.rs:2918-2950
    b[1] = 0x3C
    assert abs(_y(IQ2_XS, b, ones) - 256.0) < 1.0
    b[66] = 0x5F
    assert _y(IQ2_XS, b, ones) > 256.0


def encode(dtype, g):
    """One random block and the element values its fields define."""
    d = np.float16(g.uniform(0.001, 0.01))
    df = np.float32(d)
    e = np.zeros(256, np.float32)
    if dtype == IQ2_XXS:
        b = np.zeros(66, np.uint8)
        for ib in range(8):
            idx = g.integers(0, 256, 4)
            sidx = g.integers(0, 128, 4)
            sc = int(g.integers(0, 16))
            a1 = int(sum(int(sidx[l]) << (7 * l) for l in range(4))) | (sc << 28)
            b[2 + 8 * ib:6 + 8 * ib] = idx.astype(np.uint8)
            b[6 + 8 * ib:10 + 8 * ib] = np.frombuffer(a1.to_bytes(4, "little"), np.uint8)
            db = np.float32(np.float32(df * np.float32(0.5 + sc)) * np.float32(0.25))
            for l in range(4):
                gb, sg = gbytes("iq2xxs", idx[l]), ksigns(int(sidx[l]))
                for j in range(8):
                    e[ib * 32 + l * 8 + j] = np.float32(db * np.float32(gb[j])) * (-1 if sg >> j & 1 else 1)
    elif dtype == IQ2_XS:
        b = np.zeros(74, np.uint8)
        nib = g.integers(0, 16, 8)
        b[66:74 - 4] = 0
        for ib in range(8):
            b[66 + ib // 2] |= np.uint8(int(nib[ib]) << (4 * (ib % 2)))
            db = np.float32(np.float32(df * np.float32(0.5 + nib[ib])) * np.float32(0.25))
            for l in range(4):
                gi, si = int(g.integers(0, 512)), int(g.integers(0, 128))
                q = gi | (si << 9)
                b[2 + (ib * 4 + l) * 2:4 + (ib * 4 + l) * 2] = np.frombuffer(q.to_bytes(2, "little"), np.uint8)
                gb, sg = gbytes("iq2xs", gi), ksigns(si)
                for j in range(8):
                    e[ib * 32 + l * 8 + j] = np.float32(db * np.float32(gb[j])) * (-1 if sg >> j & 1 else 1)
    elif dtype == IQ3_XXS:
        b = np.zeros(98, np.uint8)
        for ib in range(8):
            idx = g.integers(0, 256, 8)
            sidx = g.integers(0, 128, 4)
            sc = int(g.integers(0, 16))
            aux = int(sum(int(sidx[l]) << (7 * l) for l in range(4))) | (sc << 28)
            b[2 + 8 * ib:10 + 8 * ib] = idx.astype(np.uint8)
            b[66 + 4 * ib:70 + 4 * ib] = np.frombuffer(aux.to_bytes(4, "little"), np.uint8)
            db = np.float32(np.float32(df * np.float32(0.5 + sc)) * np.float32(0.5))
            for l in range(4):
                sg = ksigns(int(sidx[l]))
                g1, g2 = gbytes("iq3xxs", idx[2 * l]), gbytes("iq3xxs", idx[2 * l + 1])
                for j in range(4):
                    e[ib * 32 + l * 8 + j] = np.float32(db * np.float32(g1[j])) * (-1 if sg >> j & 1 else 1)
                    e[ib * 32 + l * 8 + j + 4] = np.float32(db * np.float32(g2[j])) * (-1 if sg >> (j + 4) & 1 else 1)
    else:  # IQ3_S
        b = np.zeros(110, np.uint8)
        nib = g.integers(0, 16, 8)
        for ib in range(8):
            b[106 + ib // 2] |= np.uint8(int(nib[ib]) << (4 * (ib % 2)))
            db = np.float32(df * np.float32(1 + 2 * int(nib[ib])))
            idx = g.integers(0, 512, 8)
            b[2 + 8 * ib:10 + 8 * ib] = (idx & 255).astype(np.uint8)
            b[66 + ib] = np.uint8(sum(int(idx[k] >> 8) << k for k in range(8)))  # bit 2l / 2l+1
            for l in range(4):
                sg = int(g.integers(0, 256))
                b[74 + 4 * ib + l] = sg
                g1, g2 = gbytes("iq3s", idx[2 * l]), gbytes("iq3s", idx[2 * l + 1])
                for j in range(4):
                    e[ib * 32 + l * 8 + j] = np.float32(db * np.float32(g1[j])) * (-1 if sg >> j & 1 else 1)
                    e[ib * 32 + l * 8 + j + 4] = np.float32(db * np.float32(g2[j])) * (-1 if sg >> (j + 4) & 1 else 1)
    b[0:2] = np.frombuffer(d.tobytes(), np.uint8)
    return b, e


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


TYPES = [IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S]


@pytest.mark.parametrize("dtype", TYPES)
def test_layout_round_trip(dtype):
    g = np.random.default_rng(dtype)
    blocks, want = zip(*[encode(dtype, g) for _ in range(12)])
    blocks, want = np.stack(blocks), np.stack(want)
    e, rc = o.matvec_elements(dtype, blocks.reshape(-1), len(blocks), 256)
    assert rc == 0 and np.array_equal(_bits(e), _bits(want))
    for j in (0, 3, 4, 7, 100, 255):
        x = np.zeros(256, np.float32)
        x[j] = 1.0
        y, _ = o.matvec(dtype, blocks.reshape(-1), x, len(blocks), 256)
        assert np.array_equal(_bits(y + np.float32(0)), _bits(want[:, j] + np.float32(0)))


@pytest.mark.parametrize("dtype", TYPES)
def test_serial_order_and_bound(dtype):
    g = np.random.default_rng(dtype + 50)
    blocks, want = zip(*[encode(dtype, g) for _ in range(16)])
    blocks, want = np.stack(blocks), np.stack(want)
    w = blocks.reshape(-1)
    x = g.standard_normal(256).astype(np.float32)
    y, _ = o.matvec(dtype, w, x, 16, 256)
    prod = (want * x).astype(np.float32)
    order = np.arange(256)
    if dtype in (IQ3_XXS, IQ3_S):  # j, j + 4 alternating inside each group of 8
        order = np.array([g8 + j + h for g8 in range(0, 256, 8) for j in range(4) for h in (0, 4)])
    s = np.zeros(16, np.float32)
    for i in order:
        s = (s + prod[:, i]).astype(np.float32)
    assert np.array_equal(_bits(y), _bits(s))
    ex = o.matvec_exact(dtype, w, x, 16, 256)
    gam = 259 * 2.0 ** -24 / (1 - 259 * 2.0 ** -24)
    assert np.all(np.abs(y - ex) <= gam * (np.abs(want.astype(np.float64)) * np.abs(x)).sum(1))
