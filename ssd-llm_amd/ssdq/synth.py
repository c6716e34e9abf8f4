"""Seeded synthetic inputs for the quantized compute path (numpy, host side).

Distributions follow the benchmark configurations of the reference path:
  Q4_0  d ~ U[0.002, 0.02] stored as f16 (round to nearest even), 16 random
        code bytes per 32-element block (value = (q - 8) * d, streamer.rs:153-178)
  Q8_0  d ~ U[0.002, 0.02] -> f16, int8 codes uniform in [-127, 127]
  Q4_K  d, dmin ~ U[0.001, 0.01] -> f16, 12 uniform scale bytes (uniform 6-bit
        fields under the reference unpacking, compute.rs:724-731), 128 random
        code bytes
  Q6_K  d ~ U[0.001, 0.01] -> f16, random ql / qh bytes, int8 scales uniform in
        [-32, 31] (6-bit range)
  Q2_K / Q3_K / Q5_K / IQ4_NL / IQ4_XS  f16 scales ~ U[0.001, 0.01]
        (IQ4_NL U[0.002, 0.02], IQ4_XS U[0.0001, 0.001]), every other byte
        uniform random (scale fields included)
  IQ2_XXS / IQ2_XS / IQ3_XXS / IQ3_S  f16 d ~ U[0.001, 0.01], every other byte
        uniform random
  Q8_K  f32 d ~ U[0.001, 0.01], int8 codes uniform in [-127, 127], bsums the
        16-element code sums
  F16 / BF16  N(0, 0.05) rounded to the type
  activations / K / V / Q  ~ N(0, 1) f32; bf16 activations are the f32 draws
        rounded to nearest even.
Both the device path and the CPU oracle consume the same bytes, so any seeded
generator works; numpy's PCG64 keeps generation fast at full sizes.
"""
from __future__ import annotations

import numpy as np

from . import (BF16, F16, IQ2_XS, IQ2_XXS, IQ3_S, IQ3_XXS, IQ4_NL, IQ4_XS, Q2_K, Q3_K, Q4_0, Q4_K, Q5_K,
               Q6_K, Q8_0, Q8_K)

BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q2_K: (256, 84),
         Q3_K: (256, 110), Q5_K: (256, 176), Q8_K: (256, 292), IQ4_NL: (32, 18),
         IQ4_XS: (256, 148), F16: (1, 2), BF16: (1, 2), IQ2_XXS: (256, 66), IQ2_XS: (256, 74),
         IQ3_XXS: (256, 98), IQ3_S: (256, 110)}


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def _f16_bytes(vals: np.ndarray) -> np.ndarray:
    return vals.astype(np.float16).view(np.uint8).reshape(-1, 2)


def quant_weights(dtype: int, out_dim: int, in_dim: int, seed: int) -> np.ndarray:
    """Raw GGUF blocks for an out_dim x in_dim matrix, shape [out_dim * row_bytes] uint8."""
    bs, bb = BLOCK[dtype]
    nb = out_dim * (in_dim // bs)
    g = rng(seed)
    blk = np.empty((nb, bb), np.uint8)
    if dtype == Q4_0:
        blk[:, 0:2] = _f16_bytes(g.uniform(0.002, 0.02, nb).astype(np.float32))
        blk[:, 2:18] = g.integers(0, 256, (nb, 16), dtype=np.uint8)
    elif dtype == Q8_0:
        blk[:, 0:2] = _f16_bytes(g.uniform(0.002, 0.02, nb).astype(np.float32))
        blk[:, 2:34] = g.integers(-127, 128, (nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    elif dtype == Q4_K:
        blk[:, 0:2] = _f16_bytes(g.uniform(0.001, 0.01, nb).astype(np.float32))
        blk[:, 2:4] = _f16_bytes(g.uniform(0.001, 0.01, nb).astype(np.float32))
        blk[:, 4:144] = g.integers(0, 256, (nb, 140), dtype=np.uint8)
    elif dtype == Q6_K:
        blk[:, 0:192] = g.integers(0, 256, (nb, 192), dtype=np.uint8)
        blk[:, 192:208] = g.integers(-32, 32, (nb, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
        blk[:, 208:210] = _f16_bytes(g.uniform(0.001, 0.01, nb).astype(np.float32))
    elif dtype in (Q2_K, Q5_K):  # d, dmin first
        blk[:, 0:2] = _f16_bytes(g.uniform(0.001, 0.01, nb).astype(np.float32))
        blk[:, 2:4] = _f16_bytes(g.uniform(0.001, 0.01, nb).astype(np.float32))
        blk[:, 4:] = g.integers(0, 256, (nb, bb - 4), dtype=np.uint8)
    elif dtype == Q3_K:  # d last
        blk[:, 0:108] = g.integers(0, 256, (nb, 108), dtype=np.uint8)
        blk[:, 108:110] = _f16_bytes(g.uniform(0.001, 0.01, nb).astype(np.float32))
    elif dtype == Q8_K:
        blk[:, 0:4] = g.uniform(0.001, 0.01, nb).astype(np.float32).view(np.uint8).reshape(-1, 4)
        q = g.integers(-127, 128, (nb, 256), dtype=np.int16)
        blk[:, 4:260] = q.astype(np.int8).view(np.uint8)
        blk[:, 260:292] = q.reshape(nb, 16, 16).sum(axis=2).astype(np.int16).view(np.uint8)
    elif dtype in (IQ4_NL, IQ4_XS):
        lo, hi = (0.002, 0.02) if dtype == IQ4_NL else (0.0001, 0.001)
        blk[:, 0:2] = _f16_bytes(g.uniform(lo, hi, nb).astype(np.float32))
        blk[:, 2:] = g.integers(0, 256, (nb, bb - 2), dtype=np.uint8)
    elif dtype in (IQ2_XXS, IQ2_XS, IQ3_XXS, IQ3_S):  # d first, every other byte random
        blk[:, 0:2] = _f16_bytes(g.uniform(0.001, 0.01, nb).astype(np.float32))
        blk[:, 2:] = g.integers(0, 256, (nb, bb - 2), dtype=np.uint8)
    elif dtype in (F16, BF16):
        v = (g.standard_normal(nb, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
        bits = v.astype(np.float16).view(np.uint16) if dtype == F16 else f32_to_bf16_bits(v)
        return bits.view(np.uint8).reshape(-1)
    else:
        raise ValueError(f"unsupported dtype {dtype}")
    return blk.reshape(-1)


def normal_f32(shape, seed: int) -> np.ndarray:
    return rng(seed).standard_normal(shape, dtype=np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (b >> 16) & 1
    r = ((b + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def block_tables(n_seq: int, blocks_per_seq: int, seed: int, n_phys: int | None = None):
    """Random permutation of the physical blocks, [n_seq, blocks_per_seq] int32."""
    n_phys = n_phys or n_seq * blocks_per_seq
    perm = rng(seed).permutation(n_phys).astype(np.int32)
    return perm[: n_seq * blocks_per_seq].reshape(n_seq, blocks_per_seq)


def slot_mapping(tables: np.ndarray, ctx_lens, block_size: int) -> np.ndarray:
    """Pool row of every (sequence, position) in order: table[p // bs] * bs + p % bs."""
    out = []
    for s, n in enumerate(ctx_lens):
        p = np.arange(n)
        out.append(tables[s, p // block_size].astype(np.int64) * block_size + p % block_size)
    return np.concatenate(out).astype(np.int32) if out else np.zeros(0, np.int32)


# Seeds per configuration (stable across tests and the benchmark)
def seed(config: int, tensor: int) -> int:
    return 0x55D00000 + 16 * config + tensor


# byte offsets of the f16 super-block scales (d, dmin) inside one block
SCALE_FIELDS = {Q4_0: (0,), Q8_0: (0,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,)}


def signed_blocks(dtype: int, raw: np.ndarray, shift: int, seed: int) -> np.ndarray:
    """The same blocks with their f16 scales times +-2^-shift, the sign drawn
    per block and shared by the block's scales (which negates every element
    of the block).  quant_weights' Q4_K blocks have a positive mean element;
    with random signs the weights are zero-mean, as trained ones are, so that
    chained projections of O(1) inputs stay O(1) (a decoder layer)."""
    bb = BLOCK[dtype][1]
    b = raw.reshape(-1, bb).copy()
    sign = np.where(rng(seed).random(len(b)) < 0.5, -1.0, 1.0).astype(np.float16)
    for off in SCALE_FIELDS[dtype]:
        f = np.ascontiguousarray(b[:, off:off + 2]).view(np.float16)[:, 0]
        b[:, off:off + 2] = (f * (sign * np.float16(2.0 ** -shift)))[:, None].view(np.uint8)
    return b.ravel()


def decoder_layer(n_embd: int, n_head: int, n_kv: int, head_dim: int, n_ff: int, types: dict, seed: int):
    """Projections of one decoder layer as {GGUF suffix: (dtype, (in, out), raw)}
    with zero-mean blocks scaled so that each projection maps O(1) inputs to
    O(1) outputs (attn_k one more power of two down: the softmax spreads over
    a few to a few tens of positions)."""
    q_dim, kv_dim = n_head * head_dim, n_kv * head_dim
    shapes = {"attn_q": (n_embd, q_dim), "attn_k": (n_embd, kv_dim), "attn_v": (n_embd, kv_dim),
              "attn_output": (q_dim, n_embd), "ffn_gate": (n_embd, n_ff), "ffn_up": (n_embd, n_ff),
              "ffn_down": (n_ff, n_embd)}
    out = {}
    for i, (name, (k_in, n_out)) in enumerate(shapes.items()):
        dt = types[name]
        shift = int(np.ceil(np.log2(k_in) / 2)) + (1 if name == "attn_k" else 0)
        out[name] = (dt, (k_in, n_out), signed_blocks(dt, quant_weights(dt, n_out, k_in, seed + i), shift,
                                                      seed + 100 + i))
    return out
