"""Writes tests/golden/golden.json: small input/output vectors of the quantized
path, computed by the CPU oracle (oracle/, the C restatement of the reference),
plus the reference's own known-answer cases and SHA-256 digests of the
full-size bit-exact outputs.  Run from the repository root after building the
oracle:  python tests/golden/make_golden.py

Inputs are stored verbatim (hex / float bit patterns), so the fixtures do not
depend on the synthetic generator staying stable; the full-size digests also
record the digest of their generated input."""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "ssd-llm_amd")]
import ssdq_oracle as o  # noqa: E402
from ssdq import Q4_0, Q8_0, Q4_K, Q6_K, synth  # noqa: E402

BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32).tolist()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def f16_one():
    return np.array([1.0], np.float16).view(np.uint8).tolist()


def main():
    g = {"generator": "tests/golden/make_golden.py", "kats": [], "matvec": [], "int8": {},
         "paged_attention": {}, "digests": []}

    # Known answers of the reference's own tests, restated as data.
    one = f16_one()
    g["kats"].append({"name": "matvec_q4_0 all 0x88 nibbles, d=1, x=1 -> 0",
                      "source": "src/metal/compute.rs:2347-2366", "dtype": Q4_0, "out_dim": 1,
                      "in_dim": 32, "w_hex": bytes(one + [0x88] * 16).hex(), "x": [1.0] * 32,
                      "y": [0.0], "abs_tol": 1e-5})
    g["kats"].append({"name": "matvec_q8_0 d=1, codes 1, x=1 -> 32",
                      "source": "src/metal/compute.rs:2369-2381", "dtype": Q8_0, "out_dim": 1,
                      "in_dim": 32, "w_hex": bytes(one + [1] * 32).hex(), "x": [1.0] * 32,
                      "y": [32.0], "abs_tol": 1e-3})

    # Small per-type cases: 3 rows x 2 blocks, outputs from the oracle.
    for dt in (Q4_0, Q8_0, Q4_K, Q6_K):
        bs, _ = BLOCK[dt]
        out_dim, in_dim = 3, 2 * bs
        w = synth.quant_weights(dt, out_dim, in_dim, 0x601D + dt)
        x = synth.normal_f32(in_dim, 0x601D + 100 + dt)
        deq, _ = o.dequantize(dt, w, out_dim * in_dim)
        y, _ = o.matvec(dt, w, x, out_dim, in_dim)
        g["matvec"].append({"dtype": dt, "name": NAMES[dt], "out_dim": out_dim, "in_dim": in_dim,
                            "w_hex": w.tobytes().hex(), "x_bits": bits(x),
                            "dequant_bits": bits(deq), "y_bits": bits(y)})

    # INT8 rows: random, zero row, exact ties, one huge element, a negative-max row.
    dim = 16
    rows = [synth.normal_f32(dim, 0x601D + 200)]
    rows.append(np.zeros(dim, np.float32))
    rows.append(np.array([127.0, 0.5, -0.5, 1.5, -2.5, 63.5] + [0.0] * 10, np.float32))
    rows.append(np.array([1e30] + [1.0] * 15, np.float32))
    rows.append(np.array([-3.0, 1.0, 2.0] + [0.25] * 13, np.float32))
    data = np.stack(rows).astype(np.float32)
    codes, scales = o.quantize_rows(data, data.shape[0], dim)
    back = o.dequantize_rows(codes, scales, data.shape[0], dim)
    g["int8"] = {"source": "src/ssd/block_swap.rs:36-74", "dim": dim, "n_rows": data.shape[0],
                 "data_bits": bits(data), "codes": codes.astype(int).tolist(),
                 "scale_bits": bits(scales), "dequant_bits": bits(back)}

    # One 64-token paged INT8 attention case (2 sequences, GQA 4/2, hd 64, block 16).
    n_seq, n_head, n_kv, hd, bs, mb = 2, 4, 2, 64, 16, 5
    ctx = np.array([64, 23], np.int32)
    rng = np.random.default_rng(0x601D + 300)
    tables = synth.block_tables(n_seq, mb, 0x601D + 301)
    rows_n = n_seq * mb * bs
    kf = rng.standard_normal((rows_n, n_kv * hd), dtype=np.float32)
    vf = rng.standard_normal((rows_n, n_kv * hd), dtype=np.float32)
    kc, ks = o.quantize_rows(kf, rows_n, n_kv * hd)
    vc, vs = o.quantize_rows(vf, rows_n, n_kv * hd)
    q = rng.standard_normal((n_seq, n_head, hd), dtype=np.float32)
    out = o.paged_attention_int8(q, kc, ks, vc, vs, tables, ctx, n_seq, n_head, n_kv, hd, bs, mb)
    g["paged_attention"] = {
        "source": "flash_attention.rs:70-139 + paged_attention.rs:113-123 + quantized_kv_cache.rs:49-53",
        "n_seq": n_seq, "n_head": n_head, "n_head_kv": n_kv, "head_dim": hd, "block_size": bs,
        "max_blocks_per_seq": mb, "ctx_lens": ctx.tolist(), "block_tables": tables.ravel().tolist(),
        "q_bits": bits(q), "k_codes": kc.astype(int).tolist(), "k_scale_bits": bits(ks),
        "v_codes": vc.astype(int).tolist(), "v_scale_bits": bits(vs), "out_bits": bits(out)}

    # Digests of full-size bit-exact dequant outputs at the benchmark shapes.
    for dt, rows_, cols, cfg in ((Q4_0, 4096, 4096, 1), (Q8_0, 11008, 4096, 2),
                                 (Q4_K, 14336, 4096, 3), (Q6_K, 4096, 14336, 3)):
        w = synth.quant_weights(dt, rows_, cols, synth.seed(cfg, 0))
        deq, _ = o.dequantize(dt, w, rows_ * cols)
        g["digests"].append({"what": f"dequant {NAMES[dt]} {rows_}x{cols}", "dtype": dt,
                             "rows": rows_, "cols": cols, "seed": synth.seed(cfg, 0),
                             "input_sha256": sha(w), "output_sha256": sha(deq)})

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.json")
    with open(path, "w") as f:
        json.dump(g, f, separators=(",", ":"))
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
